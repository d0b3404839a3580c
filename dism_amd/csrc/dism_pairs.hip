// dism_pairs.hip -- bigram pairs: the corrections of matches with L >= 2.
//
// A valid pair (j <= i, iq[i] == ik[j]) has L >= 2 exactly when i, j >= 1 and
// iq[i-1] == ik[j-1], i.e. when the (previous label, label) bigrams of i and j are equal.
// Bigram orders (dism_sort.hip) make each bigram group one contiguous, position-ascending
// range, so the owner of a lane (a query row, or a key) finds its partners with two binary
// searches and visits only them.  Each pair's length comes from the suffix walk (bounded by
// the composed carry boundary when one is given).  Random labels give ~1/alphabet^2 of the
// causal pairs here, so these kernels carry little work next to the label scans.
//
// Mapping: lane = one owner in bigram order (neighbouring lanes usually share a group, so
// their partner loads coincide); per-lane loops over the owner's partners.
// fp32 sequences (repeated by the CPU model):
//   forward, per row: m = max(0, LUT[1], LUT[L] over pairs); p1 = exp2(LUT[1]-m);
//     ascending j: p = exp2(LUT[L]-m); dp += p; s = chain(sq.sk); c = (p - p1)*s;
//     corr[d] = fma(c, v_j[d], corr[d])
//   backward rows (l2 = lse2_i, cc = G[i+1]): P1 = exp2(LUT[1]-l2); q1 = P1*(G[1]-cc);
//     ascending j: p = exp2(LUT[L]-l2); dp = p-P1; s, e = chains; g = G[L]-cc;
//     a = p*g - q1; cdq[r] = fma(dp*e, sk[r], cdq[r]); cu = fma(dp*s, e, cu); cvv += a;
//     cw = fma(a, s*e, cw); cz += dp
//   backward keys, ascending i: p = exp2(LUT[L]-l2_i); dp = p - exp2(LUT[1]-l2_i);
//     cdk[r] = fma(dp*e, sq_i[r], cdk[r]); cdv[d] = fma(dp*s, dO_i[d], cdv[d])
#include "dism_path.h"

namespace dism {

constexpr int PAIR_ITEM = 64;

// Owner lane setup shared by the kernels: the owner's position and its partner range in the
// other side's bigram order (empty when the owner cannot have pairs).
struct Owner {
    int bh, b, h, t, p, lo, hi;
    long so, row0;
};

__device__ __forceinline__ bool pair_owner(const PathArgs& a, int side, int item_per_lane,
                                           Owner& w) {
    const int n = a.n;
    const int per = (n + PAIR_ITEM - 1) / PAIR_ITEM;
    w.bh = item_per_lane / per;
    if (w.bh >= a.B * a.H) return false;
    w.t = (item_per_lane - w.bh * per) * PAIR_ITEM + (int)threadIdx.x;
    if (w.t >= n) return false;
    w.b = w.bh / a.H;
    w.h = w.bh - w.b * a.H;
    w.so = (long)w.bh * n;
    w.row0 = (long)w.b * n * a.H + w.h;
    w.p = a.o.bpos[side][w.so + w.t];
    w.lo = w.hi = 0;
    if (a.hard[w.bh] && w.p >= 1) {
        const int other = 1 - side;
        bigram_range(a.o.bplab[other] + w.so, a.o.blab[other] + w.so,
                     a.o.btab[other] + (long)w.bh * 257, a.o.shift[w.bh],
                     (uint32_t)a.o.bplab[side][w.so + w.t], (uint32_t)a.o.blab[side][w.so + w.t],
                     w.lo, w.hi);
    }
    return true;
}

// ---------------------------------------------------------------------------------------
// forward, pass 1 per query row: pair count, row shift m, longest match (ties -> largest j),
// partner range.  grid = BH * ceil(N/64)
template <typename T, int R, int DV>
__global__ __launch_bounds__(64) void pairs_stats_kernel(PathArgs a) {
    Owner w;
    if (!pair_owner(a, 0, xcd_work_item(), w)) return;
    const int n = a.n, i = w.p;
    const int32_t* kb = a.o.bpos[1] + w.so;
    const int32_t* q = a.iq + w.so;
    const int32_t* k = a.ik + w.so;
    const int32_t* bnd = bound_of(a, w.bh);
    const float* lut = a.lut + (long)w.h * a.lut_stride;
    const float lut1 = lut[1];
    float m = lut1 > 0.0f ? lut1 : 0.0f;
    int nb = 0, best = 0, bj = -1;
    int lo = w.lo;
    while (lo < w.hi && kb[lo] == 0) ++lo;
    for (int x = lo; x < w.hi; ++x) {
        const int j = kb[x];
        if (j > i) break;
        const int L = match_length(q, k, i, j, bnd, a.strip, n);
        const float lw = lut[L];
        m = lw > m ? lw : m;
        if (L >= best) { best = L; bj = j; }
        ++nb;
    }
    a.pnb[w.so + i] = nb;
    if (nb == 0) return;
    float* rec = a.prow + (w.so + i) * a.prow_stride;
    rec[PREC_M] = m;
    rec[PREC_LB] = __int_as_float(best);
    rec[PREC_JB] = __int_as_float(bj);
    rec[PREC_LO] = __int_as_float(lo);
    rec[PREC_HI] = __int_as_float(lo + nb);
}

// ---------------------------------------------------------------------------------------
// forward, pass 2 for rows with pairs (after the label scan wrote y and the key count):
//   p1 = exp2(LUT[1]-m); ascending j: p = exp2(LUT[L]-m); dp += p; s = chain(sq.sk);
//   c = (p - p1)*s; corr[d] = fma(c, v_j[d], corr[d])
//   den = (exp2(-m) + (float)(cnt - nb)*p1) + dp; out[d] = fma(p1, y[d], corr[d]) * (1/den).
// grid = BH * ceil(N/64) * (DV/DVB)
template <typename T, int R, int DV, int DVB>
__global__ __launch_bounds__(64) void pairs_finish_kernel(PathArgs a) {
    constexpr int NBLK = DV / DVB;
    const int item = xcd_work_item();
    const int blk = item % NBLK;
    const int n = a.n, lane = threadIdx.x;
    const int per = (n + PAIR_ITEM - 1) / PAIR_ITEM;
    const int bh = item / NBLK / per;
    if (bh >= a.B * a.H) return;
    const int t = (item / NBLK - bh * per) * PAIR_ITEM + lane;
    if (t >= n) return;
    const long so = (long)bh * n;
    const int i = a.o.bpos[0][so + t];
    const int nb = a.pnb[so + i];
    if (nb == 0) return;
    const int b = bh / a.H, h = bh - b * a.H;
    const long row0 = (long)b * n * a.H + h;
    const float* rec = a.prow + (so + i) * a.prow_stride;
    const float m = rec[PREC_M];
    const int cnt = __float_as_int(rec[PREC_CNT]);
    const int lo = __float_as_int(rec[PREC_LO]), hi = __float_as_int(rec[PREC_HI]);
    const int32_t* kb = a.o.bpos[1] + so;
    const int32_t* q = a.iq + so;
    const int32_t* k = a.ik + so;
    const int32_t* bnd = bound_of(a, bh);
    const float* lut = a.lut + (long)h * a.lut_stride;
    float sqr[R];
    load_row<T, R>(reinterpret_cast<const T*>(a.sq) + (row0 + (long)i * a.H) * R, sqr);
    const float p1 = exp2_fp32(lut[1] - m);
    float dp = 0.0f, corr[DVB];
#pragma unroll
    for (int d = 0; d < DVB; ++d) corr[d] = 0.0f;
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    for (int x = lo; x < hi; ++x) {
        const int j = kb[x];
        const int L = match_length(q, k, i, j, bnd, a.strip, n);
        const float p = exp2_fp32(lut[L] - m);
        dp = dp + p;
        float skr[R];
        const long kr = row0 + (long)j * a.H;
        load_row<T, R>(sk + kr * R, skr);
        float s = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
        const float c = (p - p1) * s;
        float vr[DVB];
        load_row<T, DVB>(v + kr * DV + blk * DVB, vr);
#pragma unroll
        for (int d = 0; d < DVB; ++d) corr[d] = __builtin_fmaf(c, vr[d], corr[d]);
    }
    const float den = (exp2_fp32(-m) + (float)(cnt - nb) * p1) + dp;
    const float rden = 1.0f / den;
    const long orow = row0 + (long)i * a.H;
    const float* y = rec + PREC_Y + blk * DVB;
    if (a.out_dtype == DTYPE_F32) {
        float* o = reinterpret_cast<float*>(a.out) + orow * DV + blk * DVB;
#pragma unroll
        for (int d = 0; d < DVB; ++d) o[d] = __builtin_fmaf(p1, y[d], corr[d]) * rden;
    } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + orow * DV + blk * DVB;
#pragma unroll
        for (int d = 0; d < DVB; d += 2) {
            const uint32_t lo16 = f32_to_bf16_bits(__builtin_fmaf(p1, y[d], corr[d]) * rden);
            const uint32_t hi16 = f32_to_bf16_bits(__builtin_fmaf(p1, y[d + 1], corr[d + 1]) * rden);
            reinterpret_cast<uint32_t*>(o)[d / 2] = lo16 | (hi16 << 16);
        }
    }
    if (blk == 0) {
        a.lse2[so + i] = m + log2_fp32(den);
        if (a.lmax) a.lmax[so + i] = __float_as_int(rec[PREC_LB]);
        if (a.jarg) a.jarg[so + i] = __float_as_int(rec[PREC_JB]);
    }
}

// ---------------------------------------------------------------------------------------
// backward rows: grid = BH * ceil(N/64)
template <typename T, int R, int DV>
__global__ __launch_bounds__(64) void pairs_rows_kernel(PathArgs a) {
    Owner w;
    if (!pair_owner(a, 0, xcd_work_item(), w)) return;
    const int n = a.n, i = w.p, h = w.h;
    const long so = w.so, row0 = w.row0;
    int lo = w.lo;
    const int hi = w.hi;
    const int32_t* kb = a.o.bpos[1] + so;
    // skip to the first partner; rows without one are done
    while (lo < hi && kb[lo] == 0) ++lo;
    if (lo >= hi || kb[lo] > i) {
        a.pnb[so + i] = 0;
        return;
    }
    const int32_t* q = a.iq + so;
    const int32_t* k = a.ik + so;
    const int32_t* bnd = bound_of(a, w.bh);
    const float* lut = a.lut + (long)h * a.lut_stride;
    const float* glut = a.dlut + (long)h * a.lut_stride;
    const float l2 = a.lse2[so + i];
    const float cc = glut[i + 1];
    const float P1 = exp2_fp32(lut[1] - l2);
    const float q1 = P1 * (glut[1] - cc);
    const long qr = row0 + (long)i * a.H;
    float sqr[R], dor[DV];
    load_row<T, R>(reinterpret_cast<const T*>(a.sq) + qr * R, sqr);
    load_row<T, DV>(reinterpret_cast<const T*>(a.dout) + qr * DV, dor);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    float cdq[R], cu = 0.0f, cvv = 0.0f, cw = 0.0f, cz = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) cdq[r] = 0.0f;
    int nb = 0;
    for (int x = lo; x < hi; ++x) {
        const int j = kb[x];
        if (j > i) break;
        const int L = match_length(q, k, i, j, bnd, a.strip, n);
        const long kr = row0 + (long)j * a.H;
        float skr[R];
        load_row<T, R>(sk + kr * R, skr);
        float s = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
        float e = 0.0f;
        constexpr int VC = DV < 32 ? DV : 32;
#pragma unroll
        for (int d0 = 0; d0 < DV; d0 += VC) {
            float vr[VC];
            load_row<T, VC>(v + kr * DV + d0, vr);
#pragma unroll
            for (int d = 0; d < VC; ++d) e = __builtin_fmaf(dor[d0 + d], vr[d], e);
        }
        const float p = exp2_fp32(lut[L] - l2);
        const float dpv = p - P1;
        const float g = glut[L] - cc;
        const float av = p * g - q1;
        const float de = dpv * e, ds = dpv * s;
#pragma unroll
        for (int r = 0; r < R; ++r) cdq[r] = __builtin_fmaf(de, skr[r], cdq[r]);
        cu = __builtin_fmaf(ds, e, cu);
        cvv = cvv + av;
        cw = __builtin_fmaf(av, s * e, cw);
        cz = cz + dpv;
        ++nb;
    }
    a.pnb[so + i] = nb;
    float* rec = a.prow + (so + i) * a.prow_stride;
#pragma unroll
    for (int r = 0; r < R; ++r) rec[r] = cdq[r];
    rec[R] = cu;
    rec[R + 1] = cvv;
    rec[R + 2] = cw;
    rec[R + 3] = cz;
}

// ---------------------------------------------------------------------------------------
// backward keys: adds the bigram-pair corrections to dSK and dV written by the key label scan
//   ascending i: p = exp2(LUT[L]-l2_i); dp = p - exp2(LUT[1]-l2_i); s, e = chains;
//   cdk[r] = fma(dp*e, sq_i[r], cdk[r]); cdv[d] = fma(dp*s, dO_i[d], cdv[d]);
//   dsk[r] += cdk[r]; dv[d] += cdv[d].
// grid = BH * ceil(N/64) * (DV/DVB)
template <typename T, int R, int DV, int DVB>
__global__ __launch_bounds__(64) void pairs_keys_kernel(PathArgs a) {
    constexpr int NBLK = DV / DVB;
    const int item = xcd_work_item();
    const int blk = item % NBLK;
    Owner w;
    if (!pair_owner(a, 1, item / NBLK, w)) return;
    const int n = a.n, j = w.p;
    const long so = w.so, row0 = w.row0;
    const int32_t* qb = a.o.bpos[0] + so;
    int lo = w.lo;
    const int hi = w.hi;
    {  // first query at or after j
        int r = hi;
        while (lo < r) {
            const int mid = (lo + r) >> 1;
            if (qb[mid] < j) lo = mid + 1; else r = mid;
        }
    }
    if (lo >= hi) return;
    const int32_t* q = a.iq + so;
    const int32_t* k = a.ik + so;
    const int32_t* bnd = bound_of(a, w.bh);
    const float* lut = a.lut + (long)w.h * a.lut_stride;
    const float lut1 = lut[1];
    const long kr = row0 + (long)j * a.H;
    float skr[R], vr[DV];
    load_row<T, R>(reinterpret_cast<const T*>(a.sk) + kr * R, skr);
    load_row<T, DV>(reinterpret_cast<const T*>(a.v) + kr * DV, vr);
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    float cdk[R], cdv[DVB];
#pragma unroll
    for (int r = 0; r < R; ++r) cdk[r] = 0.0f;
#pragma unroll
    for (int d = 0; d < DVB; ++d) cdv[d] = 0.0f;
    for (int x = lo; x < hi; ++x) {
        const int i = qb[x];
        const int L = match_length(q, k, i, j, bnd, a.strip, n);
        const float l2 = a.lse2[so + i];
        const float p = exp2_fp32(lut[L] - l2);
        const float dpv = p - exp2_fp32(lut1 - l2);
        const long qr = row0 + (long)i * a.H;
        float sqr[R];
        load_row<T, R>(sq + qr * R, sqr);
        float s = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
        float e = 0.0f;
        float dblk[DVB];
        constexpr int VC = DV < 32 ? DV : 32;
#pragma unroll
        for (int d0 = 0; d0 < DV; d0 += VC) {
            float dr[VC];
            load_row<T, VC>(dout + qr * DV + d0, dr);
#pragma unroll
            for (int d = 0; d < VC; ++d) {
                e = __builtin_fmaf(dr[d], vr[d0 + d], e);
                const int db = d0 + d - blk * DVB;
                if (db >= 0 && db < DVB) dblk[db] = dr[d];
            }
        }
        const float de = dpv * e, ds = dpv * s;
        if (blk == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) cdk[r] = __builtin_fmaf(de, sqr[r], cdk[r]);
        }
#pragma unroll
        for (int d = 0; d < DVB; ++d) cdv[d] = __builtin_fmaf(ds, dblk[d], cdv[d]);
    }
    if (blk == 0) {
        float* g = a.dsk + kr * R;
#pragma unroll
        for (int r = 0; r < R; ++r) g[r] = g[r] + cdk[r];
    }
    float* g = a.dv + kr * DV + blk * DVB;
#pragma unroll
    for (int d = 0; d < DVB; ++d) g[d] = g[d] + cdv[d];
}

// ---------------------------------------------------------------------------------------
template <typename T, int R, int DV>
static hipError_t stats_go(const PathArgs& a, hipStream_t s) {
    long items = (long)((a.n + PAIR_ITEM - 1) / PAIR_ITEM) * a.B * a.H;
    items = (items + 7) / 8 * 8;
    hipLaunchKernelGGL((pairs_stats_kernel<T, R, DV>), dim3((unsigned)items), dim3(64), 0, s, a);
    return hipGetLastError();
}
template <typename T, int R, int DV>
static hipError_t finish_go(const PathArgs& a, hipStream_t s) {
    constexpr int DVB = DV < 64 ? DV : 64;
    long items = (long)((a.n + PAIR_ITEM - 1) / PAIR_ITEM) * a.B * a.H * (DV / DVB);
    items = (items + 7) / 8 * 8;
    hipLaunchKernelGGL((pairs_finish_kernel<T, R, DV, DVB>), dim3((unsigned)items), dim3(64), 0,
                       s, a);
    return hipGetLastError();
}
template <typename T, int R, int DV>
static hipError_t rows_go(const PathArgs& a, hipStream_t s) {
    long items = (long)((a.n + PAIR_ITEM - 1) / PAIR_ITEM) * a.B * a.H;
    items = (items + 7) / 8 * 8;
    hipLaunchKernelGGL((pairs_rows_kernel<T, R, DV>), dim3((unsigned)items), dim3(64), 0, s, a);
    return hipGetLastError();
}
template <typename T, int R, int DV>
static hipError_t keys_go(const PathArgs& a, hipStream_t s) {
    constexpr int DVB = DV < 64 ? DV : 64;
    long items = (long)((a.n + PAIR_ITEM - 1) / PAIR_ITEM) * a.B * a.H * (DV / DVB);
    items = (items + 7) / 8 * 8;
    hipLaunchKernelGGL((pairs_keys_kernel<T, R, DV, DVB>), dim3((unsigned)items), dim3(64), 0, s,
                       a);
    return hipGetLastError();
}

#define DISM_PAIRS_LAUNCHER(NAME, GO)                                                         \
    template <typename T, int R>                                                              \
    static hipError_t NAME##_dv(const PathArgs& a, int DV, hipStream_t s) {                   \
        switch (DV) {                                                                         \
            case 32: return GO<T, R, 32>(a, s);                                               \
            case 64: return GO<T, R, 64>(a, s);                                               \
            case 128: return GO<T, R, 128>(a, s);                                             \
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

DISM_PAIRS_LAUNCHER(pairs_stats, stats_go)
DISM_PAIRS_LAUNCHER(pairs_finish, finish_go)
DISM_PAIRS_LAUNCHER(pairs_rows, rows_go)
DISM_PAIRS_LAUNCHER(pairs_keys, keys_go)

}  // namespace dism
