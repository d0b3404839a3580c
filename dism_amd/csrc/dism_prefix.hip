// dism_prefix.hip -- prefix rows: the forward launcher.  The kernels and the algorithm are
// described in dism_prefix.h; the classification is dense_classify_kernel's (dism_dense.hip).
#include "dism_prefix.h"

DISM_TU_LAYOUT(prefix)

namespace dism {

hipError_t launch_prefix_forward(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {
    return prefix_launch<0>(a, R, DV, dtype, s);
}

}  // namespace dism
