// dism_pairs.hip -- bigram pairs: the corrections of matches with L >= 2.
//
// A valid pair (j <= i, iq[i] == ik[j]) has L >= 2 exactly when i, j >= 1 and
// iq[i-1] == ik[j-1], i.e. when the (previous label, label) bigrams of i and j are equal.
// Bigram orders (dism_sort.hip) make each bigram group one contiguous, position-ascending
// range, so an owner (a query row, or a key) finds its partners with binary searches and
// visits only them.  Each pair's length comes from the suffix walk (bounded by the composed
// carry boundary when one is given).
//
// Mapping (MI355X): a wave takes OWNERS = 16 consecutive owners of a bigram order, four
// lanes per owner ("slot").  The owners' partner lists are consumed in rounds of CK = 8
// partners per owner:
//   phase A  lane = (slot, sub): the round's pairs (two per lane) -- walk, exp2, dot
//            products -- with the per-pair coefficients and partner readout rows put in LDS;
//   phase B  lane = (slot, column group): each slot folds its round's pairs into its own
//            running sums in ascending partner order, all 16 owners at once (value-row
//            segments are loaded straight from HBM, one 4-pair batch at a time).
// Long partner lists of one owner take ceil(cnt/8) rounds; owners never wait for each other
// pair by pair.  The longest-match statistics are order-free maxima (LDS atomics).
// fp32 sequences (repeated by the CPU model), per owner over its pairs in ascending partner
// position:
//   forward rows: m = max(0, LUT[1], LUT[L]); p1 = exp2(LUT[1]-m); p = exp2(LUT[L]-m);
//     dp = dp + p; s = chain(sq.sk); corr[d] = fma((p - p1)*s, v_j[d], corr[d]);
//     den = (exp2(-m) + (float)(cnt - nb)*p1) + dp; out[d] = fma(p1, y[d], corr[d]) * (1/den)
//   backward rows (l2 = lse2_i, cc = G[i+1]): P1 = exp2(LUT[1]-l2); q1 = P1*(G[1]-cc);
//     p = exp2(LUT[L]-l2); dp = p-P1; s, e = chains; g = G[L]-cc; a = p*g - q1;
//     cdq[r] = fma(dp*e, sk[r], cdq[r]); cu = fma(dp*s, e, cu); cvv += a;
//     cw = fma(a, s*e, cw); cz += dp
//   backward keys: p = exp2(LUT[L]-l2_i); dp = p - exp2(LUT[1]-l2_i);
//     cdk[r] = fma(dp*e, sq_i[r], cdk[r]); cdv[d] = fma(dp*s, dO_i[d], cdv[d]);
//     dsk[r] += cdk[r]; dv[d] += cdv[d].
#include "dism_path.h"

namespace dism {

constexpr int OWNERS = 16;  // owners per wave, 4 lanes each
constexpr int CK = 8;       // partners per owner per round (2 per lane in phase A)

// Partner range of owner t of side SIDE's bigram order (0: query rows with key partners
// 1 <= j <= i; 1: keys with query partners i >= j): [lo, lo + cnt) of the other side's
// bigram order.
template <int SIDE>
__device__ __forceinline__ void partner_range(const PathArgs& a, int bh, long so, int t, int p,
                                              int& lo_out, int& cnt_out) {
    constexpr int OTHER = 1 - SIDE;
    int lo = 0, hi = 0;
    if (p >= 1) {
        bigram_range(a.o.bplab[OTHER] + so, a.o.blab[OTHER] + so,
                     a.o.btab[OTHER] + (long)bh * 257, a.o.shift[bh],
                     (uint32_t)a.o.bplab[SIDE][so + t], (uint32_t)a.o.blab[SIDE][so + t], lo,
                     hi);
        const int32_t* ob = a.o.bpos[OTHER] + so;
        if (SIDE == 0) {
            if (lo < hi && ob[lo] == 0) ++lo;  // key 0 has no predecessor
            int l = lo, r = hi;                // keys j <= i
            while (l < r) {
                const int mid = (l + r) >> 1;
                if (ob[mid] <= p) l = mid + 1; else r = mid;
            }
            hi = l;
        } else {
            int l = lo, r = hi;                // queries i >= j
            while (l < r) {
                const int mid = (l + r) >> 1;
                if (ob[mid] < p) l = mid + 1; else r = mid;
            }
            lo = l;
        }
    }
    lo_out = lo;
    cnt_out = hi - lo;
}

// Plan kernel: one lane per owner (both sides, grid = 2 * B*H * ceil(N/64) items): partner
// range, pair count per query row (pnb, by position), and the owners with partners appended
// to act[side] (one atomic per wave).
__global__ __launch_bounds__(64 * WAVES) void pair_plan_kernel(PathArgs a) {
    const int n = a.n, lane = lane_id();
    const int per = (n + 63) / 64;
    const int item = xcd_work_item();
    const int side = item & 1;
    const int bh = (item >> 1) / per;
    if (bh >= a.B * a.H) return;
    const long so = (long)bh * n;
    const int t = ((item >> 1) - bh * per) * 64 + lane;
    const bool own = t < n;
    const int tc = own ? t : n - 1;
    const int p = a.o.bpos[side][so + tc];
    int lo = 0, cnt = 0;
    if (own) {
        if (side == 0) partner_range<0>(a, bh, so, tc, p, lo, cnt);
        else partner_range<1>(a, bh, so, tc, p, lo, cnt);
        a.o.plo[side][so + t] = lo;
        a.o.pcnt[side][so + t] = cnt;
        if (side == 0) a.pnb[so + p] = cnt;
    }
    const unsigned long long m = __ballot(own && cnt > 0);
    if (m) {
        int base = 0;
        if (lane == 0) base = atomicAdd(&a.o.nact[side][bh], __popcll(m));
        base = __shfl(base, 0);
        if (own && cnt > 0) {
            const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
            a.o.act[side][so + base + __popcll(m & below)] = t;
        }
    }
}

hipError_t launch_pair_plan(const PathArgs& a, hipStream_t s) {
    const long items = 2L * ((a.n + 63) / 64) * a.B * a.H;
    hipLaunchKernelGGL(pair_plan_kernel, dim3(grid_for(items)), dim3(64 * WAVES), 0, s, a);
    return hipGetLastError();
}

struct Plan {
    bool own;    // this lane (< OWNERS) holds an owner
    int p;       // owner position
    int lo;      // first partner index in the other side's bigram order
    int cnt;     // partners
    int maxcnt;  // wave-uniform maximum of cnt
};

struct PairItem {
    int bh, b, h;
    long so, row0;
    int k0;      // first entry of the wave in act[side]
};

// Work item = (b,h) row and a block of OWNERS entries of its active-owner list; items past
// the list's end return at once.  grid = B*H * ceil(N/OWNERS) items.
template <int SIDE>
__device__ __forceinline__ bool pair_item(const PathArgs& a, PairItem& it, Plan& pl) {
    const int per = (a.n + OWNERS - 1) / OWNERS;
    const int item = xcd_work_item();
    it.bh = item / per;
    if (it.bh >= a.B * a.H || !a.hard[it.bh]) return false;
    it.k0 = (item - it.bh * per) * OWNERS;
    const int na = a.o.nact[SIDE][it.bh];
    if (it.k0 >= na) return false;
    it.b = it.bh / a.H;
    it.h = it.bh - it.b * a.H;
    it.so = (long)it.bh * a.n;
    it.row0 = (long)it.b * a.n * a.H + it.h;
    const int lane = lane_id();
    pl.own = lane < OWNERS && it.k0 + lane < na;
    const int t = a.o.act[SIDE][it.so + (pl.own ? it.k0 + lane : it.k0)];
    pl.p = a.o.bpos[SIDE][it.so + t];
    pl.lo = a.o.plo[SIDE][it.so + t];
    pl.cnt = pl.own ? a.o.pcnt[SIDE][it.so + t] : 0;
    int mx = pl.cnt;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const int v = __shfl_xor(mx, o);
        mx = v > mx ? v : mx;
    }
    pl.maxcnt = __builtin_amdgcn_readfirstlane(mx);
    return true;
}

// ---------------------------------------------------------------------------------------
// forward, pass 1 per query row: pair count, row shift m, longest match (ties -> largest j).
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void pairs_stats_kernel(PathArgs a) {
    __shared__ unsigned s_m_all[WAVES][OWNERS];
    __shared__ unsigned long long s_key_all[WAVES][OWNERS];
    auto& s_m = s_m_all[wave_id()];
    auto& s_key = s_key_all[wave_id()];
    PairItem it;
    Plan pl;
    if (!pair_item<0>(a, it, pl)) return;
    const int n = a.n, lane = lane_id();
    const int32_t* kb = a.o.bpos[1] + it.so;
    const int32_t* q = a.iq + it.so;
    const int32_t* k = a.ik + it.so;
    const int32_t* bnd = bound_of(a, it.bh);
    const float* lut = a.lut + (long)it.h * a.lut_stride;
    const float lut1 = lut[1];
    const float m0 = lut1 > 0.0f ? lut1 : 0.0f;
    if (lane < OWNERS) {
        s_m[lane] = __float_as_uint(m0);
        s_key[lane] = 0ull;
    }
    const int sl = lane >> 2, sub = lane & 3;
    const int i = __shfl(pl.p, sl), lo = __shfl(pl.lo, sl), cnt = __shfl(pl.cnt, sl);
    for (int c = 0; c < pl.maxcnt; c += CK) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int kq = c + sub + 4 * u;
            if (kq < cnt) {
                const int j = kb[lo + kq];
                const int L = match_length(q, k, i, j, bnd, a.strip, n);
                const float lw = lut[L];
                if (lw > m0) atomicMax(&s_m[sl], __float_as_uint(lw));
                atomicMax(&s_key[sl], ((unsigned long long)(unsigned)L << 32) | (unsigned)j);
            }
        }
    }
    if (pl.own && pl.cnt > 0) {
        float* rec = a.prow + (it.so + pl.p) * a.prow_stride;
        const unsigned long long key = s_key[lane];
        rec[PREC_M] = __uint_as_float(s_m[lane]);
        rec[PREC_LB] = __int_as_float((int)(key >> 32));
        rec[PREC_JB] = __int_as_float((int)(key & 0xffffffffu));
    }
}

// ---------------------------------------------------------------------------------------
// forward, pass 2 for rows with pairs (after the label scan wrote y and the key count).
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void pairs_finish_kernel(PathArgs a) {
    constexpr int CPL = DV / 4;  // value columns per lane in phase B
    __shared__ float s_cf_all[WAVES][OWNERS][CK];
    __shared__ float s_p_all[WAVES][OWNERS][CK];
    __shared__ int s_j_all[WAVES][OWNERS][CK];
    auto& s_cf = s_cf_all[wave_id()];
    auto& s_p = s_p_all[wave_id()];
    auto& s_j = s_j_all[wave_id()];
    PairItem it;
    Plan pl;
    if (!pair_item<0>(a, it, pl)) return;
    const int n = a.n, lane = lane_id();
    const int32_t* kb = a.o.bpos[1] + it.so;
    const int32_t* q = a.iq + it.so;
    const int32_t* k = a.ik + it.so;
    const int32_t* bnd = bound_of(a, it.bh);
    const float* lut = a.lut + (long)it.h * a.lut_stride;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);

    const int sl = lane >> 2, cg = lane & 3;
    const int i = __shfl(pl.p, sl), lo = __shfl(pl.lo, sl), cnt = __shfl(pl.cnt, sl);
    const float* rec = a.prow + (it.so + i) * a.prow_stride;
    const float m = cnt > 0 ? rec[PREC_M] : 0.0f;
    const float p1 = exp2_fp32(lut[1] - m);
    float sqr[R];
    load_row<T, R>(sq + (it.row0 + (long)i * a.H) * R, sqr);
    float dp = 0.0f, corr[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) corr[c] = 0.0f;

    for (int c0 = 0; c0 < pl.maxcnt; c0 += CK) {
        // phase A: pairs (slot, c0 + cg + 4u)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int kq = c0 + cg + 4 * u;
            if (kq < cnt) {
                const int j = kb[lo + kq];
                const int L = match_length(q, k, i, j, bnd, a.strip, n);
                const float p = exp2_fp32(lut[L] - m);
                float skr[R];
                load_row<T, R>(sk + (it.row0 + (long)j * a.H) * R, skr);
                float s = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
                s_cf[sl][cg + 4 * u] = (p - p1) * s;
                s_p[sl][cg + 4 * u] = p;
                s_j[sl][cg + 4 * u] = j;
            }
        }
        // phase B: slot sl folds pairs c0 .. c0+7 in order, lane = column group cg
        const int nv = cnt - c0 < CK ? cnt - c0 : CK;
#pragma unroll
        for (int h0 = 0; h0 < CK; h0 += 4) {
            float vr[4][CPL];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = s_j[sl][h0 + u];
                if (h0 + u < nv)
                    load_row<T, CPL>(v + (it.row0 + (long)j * a.H) * DV + cg * CPL, vr[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (h0 + u < nv) {
                    dp = dp + s_p[sl][h0 + u];
                    const float cf = s_cf[sl][h0 + u];
#pragma unroll
                    for (int c = 0; c < CPL; ++c) corr[c] = __builtin_fmaf(cf, vr[u][c], corr[c]);
                }
            }
        }
    }
    if (cnt > 0) {
        const int nb = cnt;
        const int kc = __float_as_int(rec[PREC_CNT]);
        const float den = (exp2_fp32(-m) + (float)(kc - nb) * p1) + dp;
        const float rden = 1.0f / den;
        const long orow = it.row0 + (long)i * a.H;
        const float* y = rec + PREC_Y + cg * CPL;
        if (a.out_dtype == DTYPE_F32) {
            float* o = reinterpret_cast<float*>(a.out) + orow * DV + cg * CPL;
#pragma unroll
            for (int c = 0; c < CPL; ++c) o[c] = __builtin_fmaf(p1, y[c], corr[c]) * rden;
        } else {
            uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + orow * DV + cg * CPL;
#pragma unroll
            for (int c = 0; c < CPL; c += 2) {
                const uint32_t w0 = f32_to_bf16_bits(__builtin_fmaf(p1, y[c], corr[c]) * rden);
                const uint32_t w1 =
                    f32_to_bf16_bits(__builtin_fmaf(p1, y[c + 1], corr[c + 1]) * rden);
                reinterpret_cast<uint32_t*>(o)[c / 2] = w0 | (w1 << 16);
            }
        }
        if (cg == 0) {
            a.lse2[it.so + i] = m + log2_fp32(den);
            if (a.lmax) a.lmax[it.so + i] = __float_as_int(rec[PREC_LB]);
            if (a.jarg) a.jarg[it.so + i] = __float_as_int(rec[PREC_JB]);
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward, query rows: row corrections [cdq[R], cu, cvv, cw, cz] and the pair count.
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void pairs_rows_kernel(PathArgs a) {
    constexpr int NF = 6;  // de, ds, e, av, se, dp
    __shared__ float s_f_all[WAVES][OWNERS][CK][NF];
    __shared__ float s_sk_all[WAVES][OWNERS][CK][R];
    auto& s_f = s_f_all[wave_id()];
    auto& s_sk = s_sk_all[wave_id()];
    PairItem it;
    Plan pl;
    if (!pair_item<0>(a, it, pl)) return;
    const int n = a.n, lane = lane_id();
    const int32_t* kb = a.o.bpos[1] + it.so;
    const int32_t* q = a.iq + it.so;
    const int32_t* k = a.ik + it.so;
    const int32_t* bnd = bound_of(a, it.bh);
    const float* lut = a.lut + (long)it.h * a.lut_stride;
    const float* glut = a.dlut + (long)it.h * a.lut_stride;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);

    const int sl = lane >> 2, cg = lane & 3;
    const int i = __shfl(pl.p, sl), lo = __shfl(pl.lo, sl), cnt = __shfl(pl.cnt, sl);
    const float l2 = a.lse2[it.so + i];
    const float cc = glut[i + 1];
    const float P1 = exp2_fp32(lut[1] - l2);
    const float q1 = P1 * (glut[1] - cc);
    const long qr = it.row0 + (long)i * a.H;
    float sqr[R];
    load_row<T, R>(sq + qr * R, sqr);
    constexpr int RL = (R + 3) / 4;  // readout rows handled per lane in phase B
    float cdq[RL], cu = 0.0f, cvv = 0.0f, cw = 0.0f, cz = 0.0f;
#pragma unroll
    for (int x = 0; x < RL; ++x) cdq[x] = 0.0f;

    for (int c0 = 0; c0 < pl.maxcnt; c0 += CK) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int kq = c0 + cg + 4 * u;
            if (kq < cnt) {
                const int j = kb[lo + kq];
                const int L = match_length(q, k, i, j, bnd, a.strip, n);
                const long kr = it.row0 + (long)j * a.H;
                float skr[R];
                load_row<T, R>(sk + kr * R, skr);
                float s = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
                float e = 0.0f;
                constexpr int VC = DV < 32 ? DV : 32;
#pragma unroll
                for (int d0 = 0; d0 < DV; d0 += VC) {
                    float dr[VC], vr[VC];
                    load_row<T, VC>(dout + qr * DV + d0, dr);
                    load_row<T, VC>(v + kr * DV + d0, vr);
#pragma unroll
                    for (int d = 0; d < VC; ++d) e = __builtin_fmaf(dr[d], vr[d], e);
                }
                const float p = exp2_fp32(lut[L] - l2);
                const float dpv = p - P1;
                const float av = p * (glut[L] - cc) - q1;
                float* f = s_f[sl][cg + 4 * u];
                f[0] = dpv * e;
                f[1] = dpv * s;
                f[2] = e;
                f[3] = av;
                f[4] = s * e;
                f[5] = dpv;
#pragma unroll
                for (int r = 0; r < R; ++r) s_sk[sl][cg + 4 * u][r] = skr[r];
            }
        }
        const int nv = cnt - c0 < CK ? cnt - c0 : CK;
        for (int u = 0; u < nv; ++u) {
            const float* f = s_f[sl][u];
            const float de = f[0];
#pragma unroll
            for (int x = 0; x < RL; ++x) {
                const int r = cg + 4 * x;
                if (r < R) cdq[x] = __builtin_fmaf(de, s_sk[sl][u][r], cdq[x]);
            }
            cu = __builtin_fmaf(f[1], f[2], cu);
            cvv = cvv + f[3];
            cw = __builtin_fmaf(f[3], f[4], cw);
            cz = cz + f[5];
        }
    }
    if (cnt > 0) {
        float* rec = a.prow + (it.so + i) * a.prow_stride;
#pragma unroll
        for (int x = 0; x < RL; ++x) {
            const int r = cg + 4 * x;
            if (r < R) rec[r] = cdq[x];
        }
        if (cg == 0) {
            rec[R] = cu;
            rec[R + 1] = cvv;
            rec[R + 2] = cw;
            rec[R + 3] = cz;
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward keys: adds the bigram-pair corrections to dSK and dV written by the key scan.
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void pairs_keys_kernel(PathArgs a) {
    constexpr int CPL = DV / 4;
    __shared__ float s_de_all[WAVES][OWNERS][CK];
    __shared__ float s_ds_all[WAVES][OWNERS][CK];
    __shared__ int s_i_all[WAVES][OWNERS][CK];
    __shared__ float s_sq_all[WAVES][OWNERS][CK][R];
    auto& s_de = s_de_all[wave_id()];
    auto& s_ds = s_ds_all[wave_id()];
    auto& s_i = s_i_all[wave_id()];
    auto& s_sq = s_sq_all[wave_id()];
    PairItem it;
    Plan pl;
    if (!pair_item<1>(a, it, pl)) return;
    const int n = a.n, lane = lane_id();
    const int32_t* qb = a.o.bpos[0] + it.so;
    const int32_t* q = a.iq + it.so;
    const int32_t* k = a.ik + it.so;
    const int32_t* bnd = bound_of(a, it.bh);
    const float* lut = a.lut + (long)it.h * a.lut_stride;
    const float lut1 = lut[1];
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);

    const int sl = lane >> 2, cg = lane & 3;
    const int j = __shfl(pl.p, sl), lo = __shfl(pl.lo, sl), cnt = __shfl(pl.cnt, sl);
    const long kr = it.row0 + (long)j * a.H;
    float skr[R];
    load_row<T, R>(sk + kr * R, skr);
    constexpr int RL = (R + 3) / 4;
    float cdk[RL], cdv[CPL];
#pragma unroll
    for (int x = 0; x < RL; ++x) cdk[x] = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) cdv[c] = 0.0f;

    for (int c0 = 0; c0 < pl.maxcnt; c0 += CK) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int kq = c0 + cg + 4 * u;
            if (kq < cnt) {
                const int i = qb[lo + kq];
                const int L = match_length(q, k, i, j, bnd, a.strip, n);
                const float l2 = a.lse2[it.so + i];
                const float p = exp2_fp32(lut[L] - l2);
                const float dpv = p - exp2_fp32(lut1 - l2);
                const long qr = it.row0 + (long)i * a.H;
                float sqr[R];
                load_row<T, R>(sq + qr * R, sqr);
                float s = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
                float e = 0.0f;
                constexpr int VC = DV < 32 ? DV : 32;
#pragma unroll
                for (int d0 = 0; d0 < DV; d0 += VC) {
                    float dr[VC], vr[VC];
                    load_row<T, VC>(dout + qr * DV + d0, dr);
                    load_row<T, VC>(v + kr * DV + d0, vr);
#pragma unroll
                    for (int d = 0; d < VC; ++d) e = __builtin_fmaf(dr[d], vr[d], e);
                }
                s_de[sl][cg + 4 * u] = dpv * e;
                s_ds[sl][cg + 4 * u] = dpv * s;
                s_i[sl][cg + 4 * u] = i;
#pragma unroll
                for (int r = 0; r < R; ++r) s_sq[sl][cg + 4 * u][r] = sqr[r];
            }
        }
        const int nv = cnt - c0 < CK ? cnt - c0 : CK;
#pragma unroll
        for (int h0 = 0; h0 < CK; h0 += 4) {
            float dr[4][CPL];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = s_i[sl][h0 + u];
                if (h0 + u < nv)
                    load_row<T, CPL>(dout + (it.row0 + (long)i * a.H) * DV + cg * CPL, dr[u]);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (h0 + u < nv) {
                    const float de = s_de[sl][h0 + u], ds = s_ds[sl][h0 + u];
#pragma unroll
                    for (int x = 0; x < RL; ++x) {
                        const int r = cg + 4 * x;
                        if (r < R) cdk[x] = __builtin_fmaf(de, s_sq[sl][h0 + u][r], cdk[x]);
                    }
#pragma unroll
                    for (int c = 0; c < CPL; ++c) cdv[c] = __builtin_fmaf(ds, dr[u][c], cdv[c]);
                }
            }
        }
    }
    if (cnt > 0) {
#pragma unroll
        for (int x = 0; x < RL; ++x) {
            const int r = cg + 4 * x;
            if (r < R) a.dsk[kr * R + r] = a.dsk[kr * R + r] + cdk[x];
        }
        float* g = a.dv + kr * DV + cg * CPL;
#pragma unroll
        for (int c = 0; c < CPL; ++c) g[c] = g[c] + cdv[c];
    }
}

// ---------------------------------------------------------------------------------------
#define DISM_PAIRS_LAUNCHER(NAME, KERNEL)                                                     \
    template <typename T, int R, int DV>                                                      \
    static hipError_t NAME##_go(const PathArgs& a, hipStream_t s) {                           \
        const long items = (long)((a.n + OWNERS - 1) / OWNERS) * a.B * a.H;                   \
        hipLaunchKernelGGL((KERNEL<T, R, DV>), dim3(grid_for(items)), dim3(64 * WAVES), 0, s, \
                           a);                                                                \
        return hipGetLastError();                                                             \
    }                                                                                         \
    template <typename T, int R>                                                              \
    static hipError_t NAME##_dv(const PathArgs& a, int DV, hipStream_t s) {                   \
        switch (DV) {                                                                         \
            case 32: return NAME##_go<T, R, 32>(a, s);                                        \
            case 64: return NAME##_go<T, R, 64>(a, s);                                        \
            case 128: return NAME##_go<T, R, 128>(a, s);                                      \
            default: return hipErrorInvalidValue;                                             \
        }                                                                                     \
    }                                                                                         \
    template <typename T>                                                                     \
    static hipError_t NAME##_r(const PathArgs& a, int R, int DV, hipStream_t s) {             \
        switch (R) {                                                                          \
            case 2: return NAME##_dv<T, 2>(a, DV, s);                                         \
            case 4: return NAME##_dv<T, 4>(a, DV, s);                                         \
            case 8: return NAME##_dv<T, 8>(a, DV, s);                                         \
            case 16: return NAME##_dv<T, 16>(a, DV, s);                                       \
            case 32: return NAME##_dv<T, 32>(a, DV, s);                                       \
            default: return hipErrorInvalidValue;                                             \
        }                                                                                     \
    }                                                                                         \
    hipError_t launch_##NAME(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {    \
        if (dtype == DTYPE_BF16) return NAME##_r<bf16_t>(a, R, DV, s);                        \
        if (dtype == DTYPE_F32) return NAME##_r<float>(a, R, DV, s);                          \
        return hipErrorInvalidValue;                                                          \
    }

DISM_PAIRS_LAUNCHER(pairs_stats, pairs_stats_kernel)
DISM_PAIRS_LAUNCHER(pairs_finish, pairs_finish_kernel)
DISM_PAIRS_LAUNCHER(pairs_rows, pairs_rows_kernel)
DISM_PAIRS_LAUNCHER(pairs_keys, pairs_keys_kernel)

}  // namespace dism
