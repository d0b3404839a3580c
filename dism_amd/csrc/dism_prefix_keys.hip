// dism_prefix_keys.hip -- prefix rows: the backward's key side launcher (its own
// translation unit, so the kernels' instantiations compile in parallel; dism_prefix.h).
#include "dism_prefix.h"

DISM_TU_LAYOUT(prefix_keys)

namespace dism {

hipError_t launch_prefix_keys(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {
    return prefix_launch<2>(a, R, DV, dtype, s);
}

}  // namespace dism
