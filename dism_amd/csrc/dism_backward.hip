// dism_backward.hip -- hard backward: dSQ + per-row tau terms (query sweep) and dV + dSK
// (key sweep), both recomputing match lengths from labels.
//
// Reference: dism_v3/src/hard_backward.cu:26-154 (quadratic key-major kernel with FP32
// atomics for dSQ and the tau moments) and :156-197 (tau reduce); math in
// dism_v3/python/flash_dism/reference/dism_v3_ref.py:108-127.
// MI355X design (dism_sweep.h): no atomics anywhere.  Every gradient element is owned by
// exactly one lane and accumulated in a fixed order, so the backward is deterministic and
// bit-reproducible.
//   query sweep, lane = row i of a bucket chunk, key records of the bucket ascending:
//     p = exp2(LUT[L] - lse2_i); s = sq_i.sk_j; e = dO_i.v_j; ps = p s; pe = p e; pse = ps e
//     g = G[L] - G[i+1]; dsq_i += pe sk_j; u += pse; vv = fma(p,g,vv); w = fma(pse,g,w); z += p
//     rowtau_i = (w - u ((vv - f c) / (z + f))) / (z + f),  f = exp2(-lse2_i), c = G[i+1]
//   key sweep, lane = key j of a bucket chunk, query records of the bucket ascending:
//     dv_j += ps dO_i;  dsk_j += pe sq_i
// followed by the fixed-order tau reduction in dism_aux.hip.  Pairs of the loop that are not
// matches contribute exact zeros.
#include "dism_launch.h"
#include "dism_sweep.h"

namespace dism {

// Dot of a per-lane fp32 row with a wave-uniform row of DV elements read from records in
// chunks of at most 32 words (ascending element order: fma-chain).
template <typename T, int DV>
__device__ __forceinline__ float uniform_dot(const float (&x)[DV], cptr<uint32_t> row) {
    constexpr int WV = words<T>(DV);
    constexpr int CW = WV < 32 ? WV : 32;
    constexpr int CE = sizeof(T) == 2 ? 2 * CW : CW;
    float e = 0.0f;
#pragma unroll
    for (int c = 0; c < WV / CW; ++c) {
        SRow<CW> w = srow_load<CW>(row + c * CW);
#pragma unroll
        for (int d = 0; d < CE; ++d) e = __builtin_fmaf(x[c * CE + d], srow_get<T>(w, d), e);
    }
    return e;
}

template <typename T, int R, int DV>
__global__ __launch_bounds__(64) void backward_rows_kernel(BackwardArgs a) {
    constexpr int WR = words<T>(R);
    const SweepCommon& c = a.c;
    Chunk ch;
    if (!locate_chunk(c, xcd_work_item(), false, ch)) return;
    const int lane = threadIdx.x, n = c.n;
    const int32_t* __restrict__ qpos = c.qpos + (long)ch.bh * n;
    cptr<int32_t> kpos = as_const(c.kpos + (long)ch.bh * n);
    const bool row_ok = lane < ch.count;
    const int i = row_ok ? qpos[ch.first + lane] : -1;
    const int maxrow = __builtin_amdgcn_readfirstlane(qpos[ch.first + ch.count - 1]);
    const long orow = ((long)ch.b * n + i) * c.H + ch.h;
    const long srow = (long)ch.bh * n + i;

    if (!c.hard[ch.bh]) {
        if (row_ok) {
#pragma unroll
            for (int r = 0; r < R; ++r) a.dsq[orow * R + r] = 0.0f;
            a.rowtau[srow] = 0.0f;
        }
        return;
    }
    const T* __restrict__ sq = reinterpret_cast<const T*>(a.sq);
    const T* __restrict__ dout = reinterpret_cast<const T*>(a.dout);
    const int32_t* __restrict__ q = c.iq + (long)ch.bh * n;
    const int32_t* __restrict__ k = c.ik + (long)ch.bh * n;
    const int32_t* __restrict__ bnd =
        c.bound ? c.bound + (long)ch.bh * ((n - 1) / c.strip) * n : nullptr;
    const float* __restrict__ lut = c.lut + (long)ch.h * c.lut_stride;
    const float* __restrict__ glut = a.dlut + (long)ch.h * c.lut_stride;
    cptr<uint32_t> recs = as_const(c.prec) + (long)ch.bh * n * c.pstride;
    const bool masked = c.bad[ch.bh] != 0;

    float sqr[R], dor[DV], dq[R];
    float l2 = 0.0f, cc = 0.0f;
    if (row_ok) {
        load_row<T, R>(sq + orow * R, sqr);
        load_row<T, DV>(dout + orow * DV, dor);
        l2 = a.lse2[srow];
        cc = glut[i + 1];
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) sqr[r] = 0.0f;
#pragma unroll
        for (int d = 0; d < DV; ++d) dor[d] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) dq[r] = 0.0f;
    float u = 0.0f, vv = 0.0f, w = 0.0f, z = 0.0f;
    const int myq = row_ok ? q[i] : 0;
    const bool has_prev = row_ok && i >= 1;
    const int qprev = has_prev ? q[i - 1] : 0;
    const float p1 = exp2_fp32(lut[1] - l2);
    const float g1 = glut[1] - cc;

    int pend;
    {
        int lo = ch.pbeg, hi = ch.pend;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (kpos[mid] <= maxrow) lo = mid + 1; else hi = mid;
        }
        pend = lo;
    }
    auto body = [&](auto masked_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        for (int t = ch.pbeg; t < pend; ++t) {
            cptr<uint32_t> r = recs + (long)t * c.pstride;
            const SRow<4> hd = srow_load<4>(r);
            const SRow<WR> skw = srow_load<WR>(r + 4);
            const int j = (int)hd.w[0];
            const bool valid = j <= i && (int)hd.w[1] == myq;
            float p = p1, g = g1;
            if (valid && has_prev && j >= 1 && (int)hd.w[2] == qprev) {
                const int L = match_length(q, k, i, j, bnd, c.strip, n);
                if (L != 1) {
                    p = exp2_fp32(lut[L] - l2);
                    g = glut[L] - cc;
                }
            }
            float sd = 0.0f;
#pragma unroll
            for (int x = 0; x < R; ++x) sd = __builtin_fmaf(sqr[x], srow_get<T>(skw, x), sd);
            const float e = uniform_dot<T, DV>(dor, r + 4 + WR);
            p = valid ? p : 0.0f;
            const float ps = p * sd;
            const float pe = valid ? p * e : 0.0f;
            const float pse = valid ? ps * e : 0.0f;
            if (!MASKED || valid) {
#pragma unroll
                for (int x = 0; x < R; ++x) dq[x] = __builtin_fmaf(pe, srow_get<T>(skw, x), dq[x]);
            }
            u = u + pse;
            vv = __builtin_fmaf(p, g, vv);
            w = __builtin_fmaf(pse, g, w);
            z = z + p;
        }
    };
    if (masked) body(std::true_type{});
    else body(std::false_type{});
    if (!row_ok) return;
#pragma unroll
    for (int x = 0; x < R; ++x) a.dsq[orow * R + x] = dq[x];
    const float fb = exp2_fp32(-l2);
    const float mass = z + fb;
    const float mean = __builtin_fmaf(-fb, cc, vv) / mass;
    a.rowtau[srow] = __builtin_fmaf(-u, mean, w) / mass;
}

// Key sweep.  DVB value dimensions of dv per wave (all of DV when it fits the registers);
// e = dO_i . v_j always runs over the full DV.
template <typename T, int R, int DV, int DVB>
__global__ __launch_bounds__(64) void backward_keys_kernel(BackwardArgs a) {
    constexpr int NBLK = DV / DVB;
    constexpr int WR = words<T>(R), WV = words<T>(DV), WB = words<T>(DVB);
    const SweepCommon& c = a.c;
    const int item = xcd_work_item();
    const int blk = item % NBLK;
    Chunk ch;
    if (!locate_chunk(c, item / NBLK, true, ch)) return;
    const int lane = threadIdx.x, n = c.n;
    const int32_t* __restrict__ kpos = c.kpos + (long)ch.bh * n;
    cptr<int32_t> qpos = as_const(c.qpos + (long)ch.bh * n);
    const bool key_ok = lane < ch.count;
    const int j = key_ok ? kpos[ch.first + lane] : 0x7FFFFFFF;
    const int minkey = __builtin_amdgcn_readfirstlane(kpos[ch.first]);
    const long krow = ((long)ch.b * n + (key_ok ? j : 0)) * c.H + ch.h;
    const int d0 = blk * DVB;

    if (!c.hard[ch.bh]) {
        if (key_ok) {
            if (blk == 0) {
#pragma unroll
                for (int r = 0; r < R; ++r) a.dsk[krow * R + r] = 0.0f;
            }
#pragma unroll
            for (int d = 0; d < DVB; ++d) a.dv[krow * DV + d0 + d] = 0.0f;
        }
        return;
    }
    const T* __restrict__ sk = reinterpret_cast<const T*>(a.sk);
    const T* __restrict__ v = reinterpret_cast<const T*>(a.v);
    const int32_t* __restrict__ q = c.iq + (long)ch.bh * n;
    const int32_t* __restrict__ k = c.ik + (long)ch.bh * n;
    const int32_t* __restrict__ bnd =
        c.bound ? c.bound + (long)ch.bh * ((n - 1) / c.strip) * n : nullptr;
    const float* __restrict__ lut = c.lut + (long)ch.h * c.lut_stride;
    cptr<uint32_t> recs = as_const(c.prec) + (long)ch.bh * n * c.pstride;
    const bool masked = c.bad[ch.bh] != 0;
    const float lut1 = lut[1];

    float skr[R], vr[DV], dk[R], dvv[DVB];
    if (key_ok) {
        load_row<T, R>(sk + krow * R, skr);
        load_row<T, DV>(v + krow * DV, vr);
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) skr[r] = 0.0f;
#pragma unroll
        for (int d = 0; d < DV; ++d) vr[d] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) dk[r] = 0.0f;
#pragma unroll
    for (int d = 0; d < DVB; ++d) dvv[d] = 0.0f;
    const int myk = key_ok ? k[j] : 0;
    const bool has_prev = key_ok && j >= 1;
    const int kprev = has_prev ? k[j - 1] : 0;

    // first query of the bucket that can be causal for some key of the chunk
    int pbeg;
    {
        int lo = ch.pbeg, hi = ch.pend;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (qpos[mid] < minkey) lo = mid + 1; else hi = mid;
        }
        pbeg = lo;
    }
    auto body = [&](auto masked_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        for (int t = pbeg; t < ch.pend; ++t) {
            cptr<uint32_t> r = recs + (long)t * c.pstride;
            const SRow<4> hd = srow_load<4>(r);
            const SRow<WR> sqw = srow_load<WR>(r + 4);
            const int i = (int)hd.w[0];
            const float l2 = __uint_as_float(hd.w[3]);
            const bool valid = j <= i && (int)hd.w[1] == myk;
            float p = exp2_fp32(lut1 - l2);
            if (valid && has_prev && i >= 1 && (int)hd.w[2] == kprev) {
                const int L = match_length(q, k, i, j, bnd, c.strip, n);
                if (L != 1) p = exp2_fp32(lut[L] - l2);
            }
            float sd = 0.0f;
#pragma unroll
            for (int x = 0; x < R; ++x) sd = __builtin_fmaf(srow_get<T>(sqw, x), skr[x], sd);
            const float e = uniform_dot<T, DV>(vr, r + 4 + WR);
            const float ps = valid ? p * sd : 0.0f;
            const float pe = valid ? p * e : 0.0f;
            if (!MASKED || valid) {
                const SRow<WB> dw = srow_load<WB>(r + 4 + WR + blk * WB);
#pragma unroll
                for (int d = 0; d < DVB; ++d) dvv[d] = __builtin_fmaf(ps, srow_get<T>(dw, d), dvv[d]);
                if (blk == 0) {
#pragma unroll
                    for (int x = 0; x < R; ++x) dk[x] = __builtin_fmaf(pe, srow_get<T>(sqw, x), dk[x]);
                }
            }
        }
    };
    if (masked) body(std::true_type{});
    else body(std::false_type{});
    if (!key_ok) return;
    float* o = a.dv + krow * DV + d0;
#pragma unroll
    for (int cc = 0; cc < DVB / 4; ++cc)
        reinterpret_cast<float4*>(o)[cc] =
            make_float4(dvv[4 * cc], dvv[4 * cc + 1], dvv[4 * cc + 2], dvv[4 * cc + 3]);
    if (blk == 0) {
#pragma unroll
        for (int x = 0; x < R; ++x) a.dsk[krow * R + x] = dk[x];
    }
}

// dv block per key-sweep wave: all of DV up to 64 elements, else 64
template <int DV>
constexpr int key_block() {
    return DV <= 64 ? DV : 64;
}

template <typename T, int R, int DV>
static hipError_t go_rows(const BackwardArgs& a, hipStream_t s) {
    long items = (long)a.c.slots * a.c.B * a.c.H;
    items = (items + 7) / 8 * 8;
    hipLaunchKernelGGL((backward_rows_kernel<T, R, DV>), dim3((unsigned)items), dim3(64), 0, s, a);
    return hipGetLastError();
}

template <typename T, int R, int DV>
static hipError_t go_keys(const BackwardArgs& a, hipStream_t s) {
    constexpr int DVB = key_block<DV>();
    long items = (long)a.c.slots * a.c.B * a.c.H * (DV / DVB);
    items = (items + 7) / 8 * 8;
    hipLaunchKernelGGL((backward_keys_kernel<T, R, DV, DVB>), dim3((unsigned)items), dim3(64), 0,
                       s, a);
    return hipGetLastError();
}

template <int WHICH, typename T, int R>
static hipError_t pick_dv(const BackwardArgs& a, int DV, hipStream_t s) {
    switch (DV) {
        case 32: return WHICH == 0 ? go_rows<T, R, 32>(a, s) : go_keys<T, R, 32>(a, s);
        case 64: return WHICH == 0 ? go_rows<T, R, 64>(a, s) : go_keys<T, R, 64>(a, s);
        case 128: return WHICH == 0 ? go_rows<T, R, 128>(a, s) : go_keys<T, R, 128>(a, s);
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
