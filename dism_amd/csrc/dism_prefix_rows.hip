// dism_prefix_rows.hip -- prefix rows: the backward's query side launcher (its own
// translation unit, so the kernels' instantiations compile in parallel; dism_prefix.h).
#include "dism_prefix.h"

DISM_TU_LAYOUT(prefix_rows)

namespace dism {

hipError_t launch_prefix_rows(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {
    return prefix_launch<1>(a, R, DV, dtype, s);
}

}  // namespace dism
