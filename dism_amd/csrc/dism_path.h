// dism_path.h -- device helpers shared by the pair kernels (dism_pairs.hip) and the label
// scan kernels (dism_scan.hip) of the hard core.
#pragma once
#include <limits.h>

#include "dism_device.h"
#include "dism_launch.h"

namespace dism {

// Kernels of the hard core run WAVES independent 64-lane waves per workgroup (fewer,
// longer-lived workgroups than one-wave launches, so the dispatcher keeps every SIMD fed);
// each wave owns one work item and its own slice of the workgroup's LDS.
constexpr int WAVES = 4;
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63); }
// (uniform across the wave: read into a scalar register, so that everything derived from it,
// row bases and LDS offsets, is scalar arithmetic)
__device__ __forceinline__ int wave_id() {
    return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}
// the same index as a vector value (the pair kernels: scalar row bases there raise the
// register count of pairs_keys_kernel past an occupancy step)
__device__ __forceinline__ int wave_id_v() { return (int)(threadIdx.x >> 6); }

// Work item of this wave with an XCD-contiguous mapping: workgroups are dispatched
// round-robin over the 8 XCDs, so consecutive work items (same (b,h) row, whose labels and
// vectors then stay in one XCD's L2) go to workgroups of one XCD.  grid is a multiple of 8.
__device__ __forceinline__ int xcd_work_item() {
    const int g = (int)gridDim.x, x = (int)blockIdx.x;
    return ((x & 7) * (g >> 3) + (x >> 3)) * WAVES + wave_id();
}

// workgroups for `items` work items
__host__ __forceinline__ unsigned grid_for(long items) {
    long blocks = (items + WAVES - 1) / WAVES;
    blocks = (blocks + 7) / 8 * 8;
    return (unsigned)blocks;
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

// start of position p's document: 0 for fixed-length rows, dstart[p] for packed layouts
__device__ __forceinline__ int doc_start(const PathArgs& a, int p) {
    return a.dstart ? a.dstart[p] : 0;
}

// lowest query position a suffix walk from query p may reach: its document start (packed
// rows) and its last query reset (prefill with resets); row offset so = bh * n
__device__ __forceinline__ int walk_lo(const PathArgs& a, long so, int p) {
    int lo = doc_start(a, p);
    if (a.wlo) {
        const int r = a.wlo[so + p];
        lo = r > lo ? r : lo;
    }
    return lo;
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

// ---------------------------------------------------------------------------------------
// LDS staging shared by the scan and pair kernels.
constexpr int WBYTES = 4096;  // one value-row window buffer

typedef __attribute__((address_space(3))) unsigned char lds_u8;
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void wait_vm0() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): window DMA and staging loads landed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// pairwise tree over the G consecutive lanes of a row group; the lane with g = 0 holds
// ((x0 + x1) + (x2 + x3)) + ...
template <int G>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (G >= 2) x = x + dpp<0xB1>(x);    // quad_perm [1,0,3,2]
    if constexpr (G >= 4) x = x + dpp<0x4E>(x);    // quad_perm [2,3,0,1]
    if constexpr (G >= 8) x = x + dpp<0x141>(x);   // row_half_mirror
    if constexpr (G >= 16) x = x + dpp<0x140>(x);  // row_mirror
    if constexpr (G >= 32) x = x + __shfl_xor(x, 16);
    if constexpr (G >= 64) x = x + __shfl_xor(x, 32);
    return x;
}

// Sums x[r] over the 64 lanes for every r at once.  The high lane bits go first (32, 16, ...,
// down to G = 64/R), each step pairing lane l with lane l ^ m and halving the values a lane
// holds (lanes with bit m set keep the upper half); then group_sum's adjacent tree runs over
// the G lanes of a group.  Lane l ends with the sum for r = l / G (complete where l % G == 0):
//   t[l] = x_r at lane l;  for m = 32, 16, ..., G: t[l] = t[l] + t[l + m] (l < m);
//   then ((t0 + t1) + (t2 + t3)) + ... over t[0 .. G).
template <int H, int M, int R>
__device__ __forceinline__ void transpose_step(float (&x)[R]) {
    if constexpr (H >= 1) {
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const float a = x[i], b = x[i + H];
            if constexpr (M == 32) {
                const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(a),
                                                                __float_as_uint(b), false, false);
                x[i] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
            } else if constexpr (M == 16) {
                const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(a),
                                                                __float_as_uint(b), false, false);
                x[i] = __uint_as_float(s[0]) + __uint_as_float(s[1]);
            } else {
                const bool up = lane_id() & M;
                const float keep = up ? b : a, send = up ? a : b;
                if constexpr (M == 8)
                    x[i] = keep + dpp<0x128>(send);  // row_ror:8 = lane ^ 8 within a row
                else
                    x[i] = keep + __shfl_xor(send, M);
            }
        }
        transpose_step<H / 2, M / 2, R>(x);
    }
}

template <int R>
__device__ __forceinline__ float lane_transpose_sum(float (&x)[R]) {
    transpose_step<R / 2, 32, R>(x);
    return group_sum<64 / R>(x[0]);
}

// LDS readers below take generic pointers into __shared__ arrays; after inlining the
// compiler sees the LDS origin and emits ds_read instructions.
// NV consecutive elements of T (aligned to NV * sizeof(T) or 16 bytes)
template <typename T, int NV>
__device__ __forceinline__ void lds_vals(const unsigned char* p, float (&out)[NV]) {
    constexpr int BYTES = NV * (int)sizeof(T);
    uint32_t w[(BYTES + 3) / 4];
    if constexpr (BYTES % 16 == 0) {
#pragma unroll
        for (int c = 0; c < BYTES / 16; ++c) {
            const uint4 x = reinterpret_cast<const uint4*>(p)[c];
            w[4 * c] = x.x; w[4 * c + 1] = x.y; w[4 * c + 2] = x.z; w[4 * c + 3] = x.w;
        }
    } else if constexpr (BYTES % 8 == 0) {
#pragma unroll
        for (int c = 0; c < BYTES / 8; ++c) {
            const uint2 x = reinterpret_cast<const uint2*>(p)[c];
            w[2 * c] = x.x; w[2 * c + 1] = x.y;
        }
    } else if constexpr (BYTES % 4 == 0) {
#pragma unroll
        for (int c = 0; c < BYTES / 4; ++c)
            w[c] = reinterpret_cast<const uint32_t*>(p)[c];
    } else {
        w[0] = *reinterpret_cast<const uint16_t*>(p);
    }
#pragma unroll
    for (int t = 0; t < NV; ++t) out[t] = word_elem<T>(w, t);
}

template <typename T>
__device__ __forceinline__ float lds_elem(const unsigned char* row, int d) {
    if constexpr (sizeof(T) == 2) {
        const uint16_t u = reinterpret_cast<const uint16_t*>(row)[d];
        return __uint_as_float((uint32_t)u << 16);
    } else {
        return reinterpret_cast<const float*>(row)[d];
    }
}

// R fp32 values at p (broadcast read when p is uniform)
// R consecutive fp32 values to global memory (16-byte stores where R allows; rows of R
// floats start at multiples of R floats)
template <int R>
__device__ __forceinline__ void store_row_f32(float* p, const float (&x)[R]) {
    if constexpr (R % 4 == 0) {
#pragma unroll
        for (int c = 0; c < R / 4; ++c)
            reinterpret_cast<float4*>(p)[c] = make_float4(x[4 * c], x[4 * c + 1], x[4 * c + 2],
                                                          x[4 * c + 3]);
    } else if constexpr (R % 2 == 0) {
#pragma unroll
        for (int c = 0; c < R / 2; ++c)
            reinterpret_cast<float2*>(p)[c] = make_float2(x[2 * c], x[2 * c + 1]);
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) p[r] = x[r];
    }
}

template <int R>
__device__ __forceinline__ void lds_row_f32(const float* p, float (&out)[R]) {
    if constexpr (R % 4 == 0) {
#pragma unroll
        for (int c = 0; c < R / 4; ++c) {
            const float4 x = reinterpret_cast<const float4*>(p)[c];
            out[4 * c] = x.x; out[4 * c + 1] = x.y; out[4 * c + 2] = x.z; out[4 * c + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) out[r] = p[r];
    }
}

template <typename T, int DV, int WB = WBYTES>
struct Geo {
    static constexpr int RB = DV * (int)sizeof(T);
    static constexpr int BYTES = WB;  // one window buffer
    static constexpr int WIN = WB / RB < 64 ? WB / RB : 64;
    static constexpr int NI = WIN * RB / 1024;
    static_assert((WIN * RB) % 1024 == 0, "window must be whole 1 KiB DMA blocks");
};

// DMA of `rows` value rows into buf: row s comes from src_of(s) (a byte pointer).
template <int RB, int NI, typename Src>
__device__ __forceinline__ void dma_rows(lds_u8* buf, int rows, Src src_of) {
    const int lane = lane_id();
    const int need = (rows * RB + 1023) / 1024;
#pragma unroll
    for (int t = 0; t < NI; ++t) {
        if (t < need) {
            const int byte = t * 1024 + lane * 16;
            int s = byte / RB;
            s = s < rows ? s : rows - 1;
            const unsigned char* src = src_of(s) + byte % RB;
            __builtin_amdgcn_global_load_lds(src, (lds_void*)(buf + t * 1024), 16, 0, 0);
        }
    }
}

}  // namespace dism
