// dism_forward.hip -- hard readout: match lengths -> log2 weights -> normalised signed readout.
//
// Reference: dism_v3/src/hard_forward.cu:28-118 (hard_forward_kernel) with
// dism_v3/include/forward/readout.cuh:16-100 (online max from 0, unit fallback, lse2).
// MI355X design: one lane per query row, keys streamed through the LDS symbol-bitmask table
// (dism_sweep.h); only verified matches do floating-point work, so the dense O(N^2) part of
// the operator is integer bit-scanning and the readout is O(matches * (R + DV)).
//
// Per row i, over matching keys j in ascending order (exact fp32 sequence):
//   L = match length; lw = LUT[L]
//   if lw > m: alpha = exp2(m - lw); den *= alpha; acc *= alpha; m = lw
//   p = exp2(lw - m); den += p; s = fma-chain(sq_i . sk_j); ps = p*s; acc = fma(ps, v_j, acc)
// out = acc / den; lse2 = m + log2(den); longest match (ties -> largest j) is also recorded.
#include "dism_launch.h"
#include "dism_sweep.h"

namespace dism {

template <typename T, int R, int DV>
__global__ __launch_bounds__(OWNERS) void forward_rows_kernel(ForwardArgs a) {
    __shared__ SweepShared sh;
    const int BH = a.B * a.H, n = a.n;
    const int tiles = (n + OWNERS - 1) / OWNERS;
    const int bh = blockIdx.x % BH;
    const int tile = tiles - 1 - (int)(blockIdx.x / BH);  // heaviest row tiles first
    const int b = bh / a.H, h = bh % a.H;
    const int i0 = tile * OWNERS;
    const int i = i0 + threadIdx.x;
    const bool row_ok = i < n;
    const long orow = ((long)b * n + i) * a.H + h;
    const long srow = (long)bh * n + i;

    if (!a.hard[bh]) {  // soft row: zero output and statistics
        if (row_ok) {
            if (a.out_dtype == DTYPE_F32) {
                float* o = reinterpret_cast<float*>(a.out) + orow * DV;
#pragma unroll
                for (int d = 0; d < DV; ++d) o[d] = 0.0f;
            } else {
                uint32_t* o = reinterpret_cast<uint32_t*>(a.out) + orow * (DV / 2);
#pragma unroll
                for (int d = 0; d < DV / 2; ++d) o[d] = 0u;
            }
            a.lse2[srow] = 0.0f;
            if (a.lmax) a.lmax[srow] = 0;
            if (a.jarg) a.jarg[srow] = -1;
        }
        return;
    }

    const T* __restrict__ sq = reinterpret_cast<const T*>(a.sq);
    const T* __restrict__ sk = reinterpret_cast<const T*>(a.sk);
    const T* __restrict__ v = reinterpret_cast<const T*>(a.v);
    const int32_t* __restrict__ q = a.iq + (long)bh * n;
    const int32_t* __restrict__ k = a.ik + (long)bh * n;
    const int32_t* __restrict__ bnd =
        a.bound ? a.bound + (long)bh * ((n - 1) / a.strip) * n : nullptr;
    const float* __restrict__ lut = a.lut + (long)h * a.lut_stride;

    float sqr[R];
    if (row_ok) load_row<T, R>(sq + orow * R, sqr);
    float acc[DV];
#pragma unroll
    for (int d = 0; d < DV; ++d) acc[d] = 0.0f;
    float m = 0.0f, den = 1.0f;
    int best = 0, bj = -1;
    const int myq = row_ok ? q[i] : 0;
    const int last = (i0 + OWNERS - 1 < n - 1) ? i0 + OWNERS - 1 : n - 1;

    for (int k0 = 0; k0 <= last; k0 += KT) {
        build_table(sh, k, k0, 0, last);
        if (!row_ok) continue;
        visit_tile(sh, myq, 0, i - k0 + 1, [&](int u) {
            const int j = k0 + u;
            const int L = match_length(q, k, i, j, bnd, a.strip, n);
            if (L >= best) { best = L; bj = j; }
            const float lw = lut[L];
            if (lw > m) {
                const float alpha = exp2_fp32(m - lw);
                den = den * alpha;
#pragma unroll
                for (int d = 0; d < DV; ++d) acc[d] = acc[d] * alpha;
                m = lw;
            }
            const float p = exp2_fp32(lw - m);
            den = den + p;
            const long krow = ((long)b * n + j) * a.H + h;
            float skr[R];
            load_row<T, R>(sk + krow * R, skr);
            float s = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
            const float ps = p * s;
            const T* vj = v + krow * DV;
#pragma unroll
            for (int c = 0; c < DV; c += 8) {
                float vv[8];
                load_row<T, 8>(vj + c, vv);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[c + e] = __builtin_fmaf(ps, vv[e], acc[c + e]);
            }
        });
    }
    if (!row_ok) return;
    if (a.out_dtype == DTYPE_F32) {
        float4* o = reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + orow * DV);
#pragma unroll
        for (int c = 0; c < DV / 4; ++c)
            o[c] = make_float4(acc[4 * c] / den, acc[4 * c + 1] / den, acc[4 * c + 2] / den,
                               acc[4 * c + 3] / den);
    } else {
        uint4* o = reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(a.out) + orow * DV);
#pragma unroll
        for (int c = 0; c < DV / 8; ++c) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = f32_to_bf16_bits(acc[8 * c + 2 * e] / den) |
                       (f32_to_bf16_bits(acc[8 * c + 2 * e + 1] / den) << 16);
            o[c] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
    a.lse2[srow] = m + log2_fp32(den);
    if (a.lmax) a.lmax[srow] = best;
    if (a.jarg) a.jarg[srow] = bj;
}

template <typename T, int R, int DV>
static hipError_t go(const ForwardArgs& a, hipStream_t s) {
    long tiles = (a.n + OWNERS - 1) / OWNERS;
    dim3 grid((unsigned)(tiles * a.B * a.H));
    hipLaunchKernelGGL((forward_rows_kernel<T, R, DV>), grid, dim3(OWNERS), 0, s, a);
    return hipGetLastError();
}

template <typename T, int R>
static hipError_t pick_dv(const ForwardArgs& a, int DV, hipStream_t s) {
    switch (DV) {
        case 32: return go<T, R, 32>(a, s);
        case 64: return go<T, R, 64>(a, s);
        case 128: return go<T, R, 128>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <typename T>
static hipError_t pick_r(const ForwardArgs& a, int R, int DV, hipStream_t s) {
    switch (R) {
        case 2: return pick_dv<T, 2>(a, DV, s);
        case 4: return pick_dv<T, 4>(a, DV, s);
        case 8: return pick_dv<T, 8>(a, DV, s);
        case 16: return pick_dv<T, 16>(a, DV, s);
        case 32: return pick_dv<T, 32>(a, DV, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_forward(const ForwardArgs& a, int R, int DV, int dtype, hipStream_t s) {
    if (dtype == DTYPE_BF16) return pick_r<bf16_t>(a, R, DV, s);
    if (dtype == DTYPE_F32) return pick_r<float>(a, R, DV, s);
    return hipErrorInvalidValue;
}

}  // namespace dism
