// dism_prefix.hip -- prefix rows: the classification (prefix_check_kernel) and the forward
// launcher.  The kernels and the algorithm are described in dism_prefix.h.
#include "dism_prefix.h"

namespace dism {

// ---------------------------------------------------------------------------------------
// Classification: dense rows (mode 1) whose label buckets each hold one label and one
// predecessor label become prefix rows (mode 4).  Slots hold (1 << 32) | label, 0 = empty.
__global__ __launch_bounds__(256) void prefix_check_kernel(const int32_t* __restrict__ iq,
                                                           const int32_t* __restrict__ ik,
                                                           int n, int32_t* __restrict__ dflag) {
    __shared__ unsigned long long s_lab[DENSE_BUCKETS], s_pred[DENSE_BUCKETS];
    const int bh = blockIdx.x, tid = threadIdx.x;
    if (dflag[bh] != 1) return;
    for (int x = tid; x < DENSE_BUCKETS; x += 256) {
        s_lab[x] = 0ull;
        s_pred[x] = 0ull;
    }
    __syncthreads();
    const int32_t* q = iq + (long)bh * n;
    const int32_t* k = ik + (long)bh * n;
    auto put = [](unsigned long long* tab, uint32_t b, unsigned long long tag) {
        unsigned long long cur = tab[b];
        if (cur == 0ull) {
            cur = atomicCAS(&tab[b], 0ull, tag);
            if (cur == 0ull) cur = tag;
        }
        return cur != tag;
    };
    bool bad = false;
    for (int base = 0; base < n; base += 256) {
        const int p = base + tid;
        if (p < n && !bad) {
#pragma unroll
            for (int side = 0; side < 2; ++side) {
                const int32_t* L = side ? k : q;
                const int32_t lab = L[p];
                const uint32_t b = px_bucket(lab);
                bad |= put(s_lab, b, (1ull << 32) | (uint32_t)lab);
                if (p >= 1) bad |= put(s_pred, b, (1ull << 32) | (uint32_t)L[p - 1]);
            }
        }
        if (__syncthreads_or(bad)) return;
    }
    if (tid == 0) dflag[bh] = 4;
}

hipError_t launch_prefix_check(const int32_t* iq, const int32_t* ik, long BH, int n,
                               int32_t* dflag, hipStream_t s) {
    hipLaunchKernelGGL(prefix_check_kernel, dim3((unsigned)BH), dim3(256), 0, s, iq, ik, n, dflag);
    return hipGetLastError();
}

hipError_t launch_prefix_forward(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {
    return prefix_launch<0>(a, R, DV, dtype, s);
}

}  // namespace dism
