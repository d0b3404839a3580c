// The codebook-label kernels (MFMA tiles, dism_vocab.hip) are not emulated.
#include "hip/hip_runtime.h"
#include "dism_launch.h"
DISM_TU_LAYOUT(vocab)
namespace dism {
hipError_t launch_vocab_argmax(const void*, const void*, long, int, int, int, int, int, int32_t*,
                               int32_t*, hipStream_t) {
    return hipErrorInvalidValue;
}
}
