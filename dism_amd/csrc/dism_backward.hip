// dism_backward.hip -- hard backward: dSQ + per-row tau terms (query sweep) and dV + dSK
// (key sweep), both recomputing match lengths from labels.
//
// Reference: dism_v3/src/hard_backward.cu:26-154 (quadratic key-major kernel with FP32
// atomics for dSQ and the tau moments) and :156-197 (tau reduce); math in
// dism_v3/python/flash_dism/reference/dism_v3_ref.py:108-127.
// MI355X design: no atomics anywhere.  Every gradient element is owned by exactly one lane
// and accumulated in a fixed order, so the backward is deterministic and bit-reproducible:
//   query sweep, lane = row i, keys j ascending:
//     p = exp2(LUT[L] - lse2_i); s = sq_i.sk_j; e = dO_i.v_j; ps = p s; pe = p e; pse = ps e
//     g = G[L] - G[i+1]; dsq_i += pe sk_j; u += pse; vv = fma(p,g,vv); w = fma(pse,g,w); z += p
//     rowtau_i = (w - u ((vv - f c) / (z + f))) / (z + f),  f = exp2(-lse2_i), c = G[i+1]
//   key sweep, lane = key j, rows i ascending:  dv_j += ps dO_i;  dsk_j += pe sq_i
// followed by the fixed-order tau reduction in dism_aux.hip.
#include "dism_launch.h"
#include "dism_sweep.h"

namespace dism {

template <typename T, int R, int DV>
__global__ __launch_bounds__(OWNERS) void backward_rows_kernel(BackwardArgs a) {
    __shared__ SweepShared sh;
    const int BH = a.B * a.H, n = a.n;
    const int tiles = (n + OWNERS - 1) / OWNERS;
    const int bh = blockIdx.x % BH;
    const int tile = tiles - 1 - (int)(blockIdx.x / BH);
    const int b = bh / a.H, h = bh % a.H;
    const int i0 = tile * OWNERS;
    const int i = i0 + threadIdx.x;
    const bool row_ok = i < n;
    const long orow = ((long)b * n + i) * a.H + h;
    const long srow = (long)bh * n + i;

    if (!a.hard[bh]) {
        if (row_ok) {
#pragma unroll
            for (int r = 0; r < R; ++r) a.dsq[orow * R + r] = 0.0f;
            a.rowtau[srow] = 0.0f;
        }
        return;
    }
    const T* __restrict__ sq = reinterpret_cast<const T*>(a.sq);
    const T* __restrict__ sk = reinterpret_cast<const T*>(a.sk);
    const T* __restrict__ v = reinterpret_cast<const T*>(a.v);
    const T* __restrict__ dout = reinterpret_cast<const T*>(a.dout);
    const int32_t* __restrict__ q = a.iq + (long)bh * n;
    const int32_t* __restrict__ k = a.ik + (long)bh * n;
    const int32_t* __restrict__ bnd =
        a.bound ? a.bound + (long)bh * ((n - 1) / a.strip) * n : nullptr;
    const float* __restrict__ lut = a.lut + (long)h * a.lut_stride;
    const float* __restrict__ glut = a.dlut + (long)h * a.lut_stride;

    float sqr[R], dor[DV], dq[R];
    float l2 = 0.0f, c = 0.0f;
    if (row_ok) {
        load_row<T, R>(sq + orow * R, sqr);
        load_row<T, DV>(dout + orow * DV, dor);
        l2 = a.lse2[srow];
        c = glut[i + 1];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) dq[r] = 0.0f;
    float u = 0.0f, vv = 0.0f, w = 0.0f, z = 0.0f;
    const int myq = row_ok ? q[i] : 0;
    const int last = (i0 + OWNERS - 1 < n - 1) ? i0 + OWNERS - 1 : n - 1;

    for (int k0 = 0; k0 <= last; k0 += KT) {
        build_table(sh, k, k0, 0, last);
        if (!row_ok) continue;
        visit_tile(sh, myq, 0, i - k0 + 1, [&](int uu) {
            const int j = k0 + uu;
            const int L = match_length(q, k, i, j, bnd, a.strip, n);
            const float p = exp2_fp32(lut[L] - l2);
            const long krow = ((long)b * n + j) * a.H + h;
            float skr[R];
            load_row<T, R>(sk + krow * R, skr);
            float s = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
            float e = 0.0f;
            const T* vj = v + krow * DV;
#pragma unroll
            for (int cc = 0; cc < DV; cc += 8) {
                float vx[8];
                load_row<T, 8>(vj + cc, vx);
#pragma unroll
                for (int t = 0; t < 8; ++t) e = __builtin_fmaf(dor[cc + t], vx[t], e);
            }
            const float ps = p * s, pe = p * e, pse = ps * e;
            const float g = glut[L] - c;
#pragma unroll
            for (int r = 0; r < R; ++r) dq[r] = __builtin_fmaf(pe, skr[r], dq[r]);
            u = u + pse;
            vv = __builtin_fmaf(p, g, vv);
            w = __builtin_fmaf(pse, g, w);
            z = z + p;
        });
    }
    if (!row_ok) return;
#pragma unroll
    for (int r = 0; r < R; ++r) a.dsq[orow * R + r] = dq[r];
    const float f = exp2_fp32(-l2);
    const float mass = z + f;
    const float mean = __builtin_fmaf(-f, c, vv) / mass;
    a.rowtau[srow] = __builtin_fmaf(-u, mean, w) / mass;
}

template <typename T, int R, int DV>
__global__ __launch_bounds__(OWNERS) void backward_keys_kernel(BackwardArgs a) {
    __shared__ SweepShared sh;
    const int BH = a.B * a.H, n = a.n;
    const int bh = blockIdx.x % BH;
    const int tile = (int)(blockIdx.x / BH);  // key tile 0 has the most rows: heaviest first
    const int b = bh / a.H, h = bh % a.H;
    const int j0 = tile * OWNERS;
    const int j = j0 + threadIdx.x;
    const bool key_ok = j < n;
    const long krow = ((long)b * n + j) * a.H + h;

    if (!a.hard[bh]) {
        if (key_ok) {
#pragma unroll
            for (int r = 0; r < R; ++r) a.dsk[krow * R + r] = 0.0f;
#pragma unroll
            for (int d = 0; d < DV; ++d) a.dv[krow * DV + d] = 0.0f;
        }
        return;
    }
    const T* __restrict__ sq = reinterpret_cast<const T*>(a.sq);
    const T* __restrict__ sk = reinterpret_cast<const T*>(a.sk);
    const T* __restrict__ v = reinterpret_cast<const T*>(a.v);
    const T* __restrict__ dout = reinterpret_cast<const T*>(a.dout);
    const int32_t* __restrict__ q = a.iq + (long)bh * n;
    const int32_t* __restrict__ k = a.ik + (long)bh * n;
    const int32_t* __restrict__ bnd =
        a.bound ? a.bound + (long)bh * ((n - 1) / a.strip) * n : nullptr;
    const float* __restrict__ lut = a.lut + (long)h * a.lut_stride;
    const float* __restrict__ l2row = a.lse2 + (long)bh * n;

    float skr[R], vr[DV], dk[R], dvv[DV];
    if (key_ok) {
        load_row<T, R>(sk + krow * R, skr);
        load_row<T, DV>(v + krow * DV, vr);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) dk[r] = 0.0f;
#pragma unroll
    for (int d = 0; d < DV; ++d) dvv[d] = 0.0f;
    const int myk = key_ok ? k[j] : 0;

    for (int q0 = j0; q0 < n; q0 += KT) {
        build_table(sh, q, q0, j0, n - 1);
        if (!key_ok) continue;
        visit_tile(sh, myk, j - q0, n - q0, [&](int uu) {
            const int i = q0 + uu;
            const int L = match_length(q, k, i, j, bnd, a.strip, n);
            const float p = exp2_fp32(lut[L] - l2row[i]);
            const long qrow = ((long)b * n + i) * a.H + h;
            float sqv[R];
            load_row<T, R>(sq + qrow * R, sqv);
            float s = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqv[r], skr[r], s);
            const float ps = p * s;
            float e = 0.0f;
            const T* doi = dout + qrow * DV;
#pragma unroll
            for (int cc = 0; cc < DV; cc += 8) {
                float dx[8];
                load_row<T, 8>(doi + cc, dx);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    e = __builtin_fmaf(dx[t], vr[cc + t], e);
                    dvv[cc + t] = __builtin_fmaf(ps, dx[t], dvv[cc + t]);
                }
            }
            const float pe = p * e;
#pragma unroll
            for (int r = 0; r < R; ++r) dk[r] = __builtin_fmaf(pe, sqv[r], dk[r]);
        });
    }
    if (!key_ok) return;
    float4* o = reinterpret_cast<float4*>(a.dv + krow * DV);
#pragma unroll
    for (int cc = 0; cc < DV / 4; ++cc)
        o[cc] = make_float4(dvv[4 * cc], dvv[4 * cc + 1], dvv[4 * cc + 2], dvv[4 * cc + 3]);
#pragma unroll
    for (int r = 0; r < R; ++r) a.dsk[krow * R + r] = dk[r];
}

template <int WHICH, typename T, int R, int DV>
static hipError_t go(const BackwardArgs& a, hipStream_t s) {
    long tiles = (a.n + OWNERS - 1) / OWNERS;
    dim3 grid((unsigned)(tiles * a.B * a.H));
    if (WHICH == 0)
        hipLaunchKernelGGL((backward_rows_kernel<T, R, DV>), grid, dim3(OWNERS), 0, s, a);
    else
        hipLaunchKernelGGL((backward_keys_kernel<T, R, DV>), grid, dim3(OWNERS), 0, s, a);
    return hipGetLastError();
}

template <int WHICH, typename T, int R>
static hipError_t pick_dv(const BackwardArgs& a, int DV, hipStream_t s) {
    switch (DV) {
        case 32: return go<WHICH, T, R, 32>(a, s);
        case 64: return go<WHICH, T, R, 64>(a, s);
        case 128: return go<WHICH, T, R, 128>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <int WHICH, typename T>
static hipError_t pick_r(const BackwardArgs& a, int R, int DV, hipStream_t s) {
    switch (R) {
        case 2: return pick_dv<WHICH, T, 2>(a, DV, s);
        case 4: return pick_dv<WHICH, T, 4>(a, DV, s);
        case 8: return pick_dv<WHICH, T, 8>(a, DV, s);
        case 16: return pick_dv<WHICH, T, 16>(a, DV, s);
        case 32: return pick_dv<WHICH, T, 32>(a, DV, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_backward_rows(const BackwardArgs& a, int R, int DV, int dtype, hipStream_t s) {
    if (dtype == DTYPE_BF16) return pick_r<0, bf16_t>(a, R, DV, s);
    if (dtype == DTYPE_F32) return pick_r<0, float>(a, R, DV, s);
    return hipErrorInvalidValue;
}

hipError_t launch_backward_keys(const BackwardArgs& a, int R, int DV, int dtype, hipStream_t s) {
    if (dtype == DTYPE_BF16) return pick_r<1, bf16_t>(a, R, DV, s);
    if (dtype == DTYPE_F32) return pick_r<1, float>(a, R, DV, s);
    return hipErrorInvalidValue;
}

}  // namespace dism
