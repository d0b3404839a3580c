// dism_forward.hip -- hard readout: match lengths -> log2 weights -> normalised signed readout.
//
// Reference: dism_v3/src/hard_forward.cu:28-118 (hard_forward_kernel) with
// dism_v3/include/forward/readout.cuh:16-100 (online max from 0, unit fallback, lse2).
// MI355X design (dism_sweep.h): one wave per (64 query rows of one label bucket, block of up
// to 64 value dimensions), lane = row, wave-uniform loop over the bucket's keys with the key
// data in scalar registers, prefetched one key ahead.  Two passes over the keys: the first
// finds the row shift m_i = max(0, max_j LUT[L_ij]) and the longest match; the second
// accumulates with m_i fixed, so no rescaling happens inside the loop.  Per row i, over
// matching keys j in ascending order (exact fp32 sequence, also the CPU model's):
//   den = exp2(-m); per match: p = exp2(LUT[L] - m); den += p; s = fma-chain(sq_i . sk_j);
//   ps = p*s; acc = fma(ps, v_j, acc)
//   out = acc / den; lse2 = m + log2(den).
// Non-matching keys of the loop contribute exact zeros (p = 0, ps = 0).  When a (b,h) row
// holds a non-finite input the accumulation is additionally guarded per lane.
// Soft (b,h) rows give zero output and statistics.
#include "dism_launch.h"
#include "dism_sweep.h"

namespace dism {

template <typename T, int R, int DV, int DVB>
__global__ __launch_bounds__(64) void forward_kernel(ForwardArgs a) {
    constexpr int NBLK = DV / DVB;
    constexpr int WR = words<T>(R), WV = words<T>(DVB);
    const SweepCommon& c = a.c;
    const int item = xcd_work_item();
    const int blk = item % NBLK;
    Chunk ch;
    if (!locate_chunk(c, item / NBLK, false, ch)) return;
    const int lane = threadIdx.x, n = c.n;
    const int32_t* __restrict__ qpos = c.qpos + (long)ch.bh * n;
    cptr<int32_t> kpos = as_const(c.kpos + (long)ch.bh * n);
    const bool row_ok = lane < ch.count;
    const int i = row_ok ? qpos[ch.first + lane] : -1;
    const int maxrow = __builtin_amdgcn_readfirstlane(qpos[ch.first + ch.count - 1]);
    const long orow = ((long)ch.b * n + i) * c.H + ch.h;
    const long srow = (long)ch.bh * n + i;
    const int d0 = blk * DVB;

    if (!c.hard[ch.bh]) {
        if (row_ok) {
            if (a.out_dtype == DTYPE_F32) {
                float* o = reinterpret_cast<float*>(a.out) + orow * DV + d0;
#pragma unroll
                for (int d = 0; d < DVB; ++d) o[d] = 0.0f;
            } else {
                uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + orow * DV + d0;
#pragma unroll
                for (int d = 0; d < DVB; ++d) o[d] = 0;
            }
            if (blk == 0) {
                a.lse2[srow] = 0.0f;
                if (a.lmax) a.lmax[srow] = 0;
                if (a.jarg) a.jarg[srow] = -1;
            }
        }
        return;
    }

    const T* __restrict__ sq = reinterpret_cast<const T*>(a.sq);
    const int32_t* __restrict__ q = c.iq + (long)ch.bh * n;
    const int32_t* __restrict__ k = c.ik + (long)ch.bh * n;
    const int32_t* __restrict__ bnd =
        c.bound ? c.bound + (long)ch.bh * ((n - 1) / c.strip) * n : nullptr;
    const float* __restrict__ lut = c.lut + (long)ch.h * c.lut_stride;
    const float lut1 = lut[1];
    const bool masked = c.bad[ch.bh] != 0;

    const int myq = row_ok ? q[i] : 0;
    const bool has_prev = row_ok && i >= 1;
    const int qprev = has_prev ? q[i - 1] : 0;

    // partner records of the bucket; the keys causal for some row of the chunk are [pbeg, pend)
    cptr<uint32_t> recs = as_const(c.prec) + (long)ch.bh * n * c.pstride;
    int pend;
    {
        int lo = ch.pbeg, hi = ch.pend;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (kpos[mid] <= maxrow) lo = mid + 1; else hi = mid;
        }
        pend = lo;
    }

    // ---- pass 1: row shift and longest match (record headers only)
    float m = 0.0f;
    int best = 0, bj = -1;
    if (ch.pbeg < pend) {
        SRow<4> cur = srow_load<4>(recs + (long)ch.pbeg * c.pstride);
        for (int t = ch.pbeg; t < pend; ++t) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): `cur` is resident
            SRow<4> nxt;
            if (t + 1 < pend) nxt = srow_load<4>(recs + (long)(t + 1) * c.pstride);
            const int j = (int)cur.w[0];
            const bool valid = j <= i && (int)cur.w[1] == myq;
            int L = 1;
            if (valid && has_prev && j >= 1 && (int)cur.w[2] == qprev)
                L = match_length(q, k, i, j, bnd, c.strip, n);
            const float lw = L == 1 ? lut1 : lut[L];
            m = (valid && lw > m) ? lw : m;
            const bool upd = valid && L >= best;
            best = upd ? L : best;
            bj = upd ? j : bj;
            cur = nxt;
        }
    }
    if (row_ok && blk == 0) {
        if (a.lmax) a.lmax[srow] = best;
        if (a.jarg) a.jarg[srow] = bj;
    }

    // ---- pass 2: accumulation with the row shift fixed
    float sqr[R];
    if (row_ok) {
        load_row<T, R>(sq + orow * R, sqr);
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) sqr[r] = 0.0f;
    }
    float den = exp2_fp32(-m);
    const float p1 = exp2_fp32(lut1 - m);
    float acc[DVB];
#pragma unroll
    for (int d = 0; d < DVB; ++d) acc[d] = 0.0f;

    struct Key {
        SRow<4> hd;
        SRow<WR> skw;
        SRow<WV> vw;
    };
    auto fetch = [&](int t) {
        Key x;
        cptr<uint32_t> r = recs + (long)t * c.pstride;
        x.hd = srow_load<4>(r);
        x.skw = srow_load<WR>(r + 4);
        x.vw = srow_load<WV>(r + 4 + WR + blk * WV);
        return x;
    };
    auto body = [&](auto masked_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        if (ch.pbeg >= pend) return;
        Key cur = fetch(ch.pbeg);
        for (int t = ch.pbeg; t < pend; ++t) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): `cur` is resident
            Key nxt;
            if (t + 1 < pend) nxt = fetch(t + 1);
            const int j = (int)cur.hd.w[0];
            const bool valid = j <= i && (int)cur.hd.w[1] == myq;
            float p = p1;
            if (valid && has_prev && j >= 1 && (int)cur.hd.w[2] == qprev) {
                const int L = match_length(q, k, i, j, bnd, c.strip, n);
                if (L != 1) p = exp2_fp32(lut[L] - m);
            }
            p = valid ? p : 0.0f;
            den = den + p;
            float sd = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) sd = __builtin_fmaf(sqr[r], srow_get<T>(cur.skw, r), sd);
            const float ps = valid ? p * sd : 0.0f;
            if (!MASKED || valid) {
#pragma unroll
                for (int d = 0; d < DVB; ++d)
                    acc[d] = __builtin_fmaf(ps, srow_get<T>(cur.vw, d), acc[d]);
            }
            cur = nxt;
        }
    };
    if (masked) body(std::true_type{});
    else body(std::false_type{});

    if (!row_ok) return;
    if (a.out_dtype == DTYPE_F32) {
        float* o = reinterpret_cast<float*>(a.out) + orow * DV + d0;
#pragma unroll
        for (int cc = 0; cc < DVB / 4; ++cc)
            reinterpret_cast<float4*>(o)[cc] =
                make_float4(acc[4 * cc] / den, acc[4 * cc + 1] / den, acc[4 * cc + 2] / den,
                            acc[4 * cc + 3] / den);
    } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + orow * DV + d0;
#pragma unroll
        for (int cc = 0; cc < DVB / 8; ++cc) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = f32_to_bf16_bits(acc[8 * cc + 2 * e] / den) |
                       (f32_to_bf16_bits(acc[8 * cc + 2 * e + 1] / den) << 16);
            reinterpret_cast<uint4*>(o)[cc] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
    if (blk == 0) a.lse2[srow] = m + log2_fp32(den);
}

template <typename T, int R, int DV>
static hipError_t go(const ForwardArgs& a, hipStream_t s) {
    constexpr int DVB = value_block<T, R, DV>();
    long items = (long)a.c.slots * a.c.B * a.c.H * (DV / DVB);
    items = (items + 7) / 8 * 8;
    hipLaunchKernelGGL((forward_kernel<T, R, DV, DVB>), dim3((unsigned)items), dim3(64), 0, s, a);
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
