// dism_path.h -- device helpers shared by the pair kernels (dism_pairs.hip) and the label
// scan kernels (dism_scan.hip) of the hard core.
#pragma once
#include <limits.h>

#include "dism_device.h"
#include "dism_launch.h"

namespace dism {

// Work-item index of this workgroup with an XCD-contiguous mapping: workgroups are dispatched
// round-robin over the 8 XCDs, so consecutive work items (same (b,h) row, whose labels and
// vectors then stay in one XCD's L2) go to workgroups of one XCD.  grid is a multiple of 8.
__device__ __forceinline__ int xcd_work_item() {
    const int g = (int)gridDim.x, x = (int)blockIdx.x;
    return (x & 7) * (g >> 3) + (x >> 3);
}

__host__ __device__ constexpr int words_of(int elem_bytes, int n) {
    return elem_bytes == 2 ? (n + 1) / 2 : n;
}

// element e of a row held as raw 32-bit words
template <typename T>
__device__ __forceinline__ float word_elem(const uint32_t* w, int e) {
    if constexpr (sizeof(T) == 2) {
        const uint32_t x = w[e >> 1];
        return (e & 1) ? bf16_hi(x) : bf16_lo(x);
    } else {
        return __uint_as_float(w[e]);
    }
}

// W raw words of a row (16/8/4-byte accesses as the row length allows; rows are aligned to
// their length's power-of-two part because every row starts at a multiple of its length)
template <int W>
__device__ __forceinline__ void load_words(const void* row, uint32_t (&w)[W]) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row);
    if constexpr (W % 4 == 0) {
#pragma unroll
        for (int c = 0; c < W / 4; ++c) {
            const uint4 x = reinterpret_cast<const uint4*>(p)[c];
            w[4 * c] = x.x; w[4 * c + 1] = x.y; w[4 * c + 2] = x.z; w[4 * c + 3] = x.w;
        }
    } else if constexpr (W % 2 == 0) {
#pragma unroll
        for (int c = 0; c < W / 2; ++c) {
            const uint2 x = reinterpret_cast<const uint2*>(p)[c];
            w[2 * c] = x.x; w[2 * c + 1] = x.y;
        }
    } else {
#pragma unroll
        for (int c = 0; c < W; ++c) w[c] = p[c];
    }
}

template <typename T>
__device__ __forceinline__ float load_elem(const T* p, long idx) {
    if constexpr (sizeof(T) == 2) {
        return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[idx] << 16);
    } else {
        return reinterpret_cast<const float*>(p)[idx];
    }
}

// first index in [lo, hi) whose unsigned label is >= x (lower) / > x (upper)
__device__ __forceinline__ int lower_label(const int32_t* lab, int lo, int hi, uint32_t x) {
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((uint32_t)lab[mid] < x) lo = mid + 1; else hi = mid;
    }
    return lo;
}
__device__ __forceinline__ int upper_label(const int32_t* lab, int lo, int hi, uint32_t x) {
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((uint32_t)lab[mid] <= x) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// bigram group (pl, cl) of the other side's bigram order: [lo, hi).  The search starts from
// that order's run of the top sorted digit of pl (btab / shift).
__device__ __forceinline__ void bigram_range(const int32_t* bplab, const int32_t* blab,
                                             const int32_t* btab, int bshift, uint32_t pl,
                                             uint32_t cl, int& lo_out, int& hi_out) {
    const unsigned long long key = ((unsigned long long)pl << 32) | cl;
    auto at = [&](int x) {
        return ((unsigned long long)(uint32_t)bplab[x] << 32) | (uint32_t)blab[x];
    };
    const int dig = (int)((pl >> bshift) & 255u);
    int lo = btab[dig], hi = btab[dig + 1];
    const int top = hi;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (at(mid) < key) lo = mid + 1; else hi = mid;
    }
    lo_out = lo;
    hi = top;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (at(mid) <= key) lo = mid + 1; else hi = mid;
    }
    hi_out = lo;
}

__device__ __forceinline__ int readlane_i(int v, int l) {
    return __builtin_amdgcn_readlane(v, l);
}
__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// sum over the 64 lanes of a wave, xor-butterfly order (32, 16, 8, 4, 2, 1); every lane
// receives the same bits
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = x + __shfl_xor(x, o);
    return x;
}

__device__ __forceinline__ const int32_t* bound_of(const PathArgs& a, int bh) {
    return a.bound ? a.bound + (long)bh * ((a.n - 1) / a.strip) * a.n : nullptr;
}

}  // namespace dism
