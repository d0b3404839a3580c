// dism_levels.hip -- level rows (mode 3): dense hard rows whose sums are taken per match
// length instead of per pair.
//
// For a valid pair (j <= i, L >= 1) the weight is p(L) = exp2(LUT[L] - m).  With
// c_l = p(l) - p(l - 1) (p(0) = 0), every sum over the valid keys of a query telescopes:
//   sum_j p(L_ij) x_j = sum over l of c_l * (sum of x_j over the keys with L_ij >= l),
// and the keys with L_ij >= l are exactly the keys before query i in its level-l group (the
// entries sharing the l-gram ending at their position; level_prep_kernel in dism_sort.hip
// builds the per-level lists, groups in position order).  So a query needs, per level, the
// prefix matrix M = sum of sk_j (x) v_j over its group's keys before it -- an R x DV fma
// chain -- instead of R + DV work per pair: for a small alphabet (d_qk = 2) there are about
// log4(N) levels but N/4 valid keys per query.  The same holds for the backward: the query
// side reads dO . M (its dq, u, w terms), the key side the suffix matrix of c_l sq_i (x) dO_i
// over the queries after it in its group.
//
// Level lists are cut into segments of LEVEL_SEG entries.  level_tot_kernel forms, per
// segment whose last group piece continues into the next segment, that piece's key sum T_s
// (one wave per segment); a segment's prefix is then P_s = ((T_{s0} + T_{s0+1}) + ...) +
// T_{s-1} over the segments since its first group began (P_{s+1} = P_s + T_s, P_{s0+1} =
// T_{s0}).  level_scan_kernel walks every segment with one wave: M starts from the
// segment's P (when its first group began in an earlier segment), restarts at zero at each
// group start, adds each key and is read by each query (its y_l, or z_l in the backward)
// into a per-entry buffer.  The key side mirrors this (U_s over a segment's first piece,
// Q_{s-1} = Q_s + U_s, the walk in descending order, dv_l and dk_l per key entry).  The
// combine kernels then sum each query's (key's) levels in ascending order.
//
// Lanes = value columns (DV <= 128: CPL = 1 or 2 per lane) in the walks: a segment's 32
// entries are loaded at once (their rows by the entry's own lane, broadcast with readlane;
// their value / gradient columns by every lane), then the walk runs in registers.
// Everything is a fixed fp32 sequence, restated by the oracle's level_forward_row /
// level_backward_row (oracle/dism_cpu_model.c):
//   forward, query i: m = max(0, LUT[l] over the lengths present, n_l > n_{l+1});
//     den = exp2(-m); for l = 1..Lq: den = fma(c_l, n_l, den);
//     acc[d] = fma(c_l, y_l[d], acc[d]), y_l[d] = chain_r fma(sq[r], M[r][d]);
//     out = acc / den; lse2 = m + log2(den).
//   backward rows (p_l from lse2): z_l[r] = lane tree of dO[d] M[r][d]; w_l = chain_r
//     fma(sq[r], z_l[r]); F_l = p_l (G[l] - G[i+1]), dF_l = F_l - F_{l-1};
//     dq[r] = fma(c_l, z_l[r], dq[r]); u = fma(c_l, w_l, u); vv = fma(dF_l, n_l, vv);
//     ww = fma(dF_l, w_l, ww); z = fma(c_l, n_l, z).
//   backward keys, key j, level l: K[d][r] = fma(c_l(i) sq_i[r], dO_i[d], K) over the
//     queries after it in its piece, descending, from Q or 0; dv_l[d] = chain_r
//     fma(sk[r], K[d][r]); dk_l[r] = lane tree of v[d] K[d][r]; dv = dv_1 + dv_2 + ...
// The lane tree: lane t holds its columns' chain (t, then t + 64), lanes without a column
// hold +0, then x = x + shfl_xor(x, o) for o = 32, 16, ..., 1.
#include "dism_path.h"

DISM_TU_LAYOUT(levels)

namespace dism {

constexpr int LV_THREADS = 256;
constexpr int LV_WAVES = LV_THREADS / 64;
constexpr unsigned LV_GRID = 1024;    // persistent workgroups of the combine kernels
constexpr int LV_MAX_SEGS = 2 * LEVEL_MAX_N / LEVEL_SEG;  // segments of one level list

template <typename T>
__device__ __forceinline__ float elem(const T* p) {
    if constexpr (sizeof(T) == 2)
        return __uint_as_float((uint32_t)(*reinterpret_cast<const uint16_t*>(p)) << 16);
    else
        return *p;
}

__device__ __forceinline__ float lane_tree(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = x + __shfl_xor(x, o);
    return x;
}

// N consecutive fp32 values (rows of N floats start at multiples of N floats)
template <int N>
__device__ __forceinline__ void store_f32_row_l(float* o, const float (&x)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int c = 0; c < N / 4; ++c)
            reinterpret_cast<float4*>(o)[c] = make_float4(x[4 * c], x[4 * c + 1], x[4 * c + 2],
                                                          x[4 * c + 3]);
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (int c = 0; c < N / 2; ++c)
            reinterpret_cast<float2*>(o)[c] = make_float2(x[2 * c], x[2 * c + 1]);
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) o[c] = x[c];
    }
}

__device__ __forceinline__ int rl(int x, int t) { return __builtin_amdgcn_readlane(x, t); }
__device__ __forceinline__ float rlf(float x, int t) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), t));
}
__device__ __forceinline__ int lv_e(int x) { return x & LEVEL_EMASK; }
__device__ __forceinline__ int lv_n(int x) { return (x >> LEVEL_EBITS) & LEVEL_EMASK; }

// per-row views of the level state
struct LvRow {
    const int32_t* ent;   // the row's level lists (level l at (l - 1) 2n)
    const int32_t* meta;
    int bh, b, h, n;
    long so, row0, ebase;  // ebase: the row's first entry slot (per-entry buffers)
    __device__ int off(int l) const { return meta[1 + l]; }  // level l+1's first entry slot
    __device__ const int32_t* list(int l) const { return ent + (long)(l - 1) * 2 * n; }
    __device__ int segbase(int l) const { return meta[LEVEL_MAX + 2 + l]; }
};

__device__ __forceinline__ LvRow lv_row(const PathArgs& a, int bh) {
    LvRow r;
    const int n = a.n;
    r.bh = bh;
    r.n = n;
    r.b = bh / a.H;
    r.h = bh - r.b * a.H;
    r.so = (long)bh * n;
    r.row0 = (long)r.b * n * a.H + r.h;
    r.ebase = (long)bh * LEVEL_BUDGET * n;
    r.ent = a.o.lvent + (long)bh * LEVEL_MAX * 2 * n;
    r.meta = a.o.lvmeta + (long)bh * LEVEL_META;
    return r;
}

// One segment of a level list held by a wave: lane t < cnt holds entry t (ev with its flags
// and count, e the entry alone), its row (sk of a key, sq of a query) in rv, and for each
// entry t every lane holds column lane + 64 c of its value row (keys) or gradient row
// (queries), as KEYCOLS / QUERYCOLS select, in col[t][c].
template <typename T, int R, int DV>
struct SegData {
    static constexpr int CPL = (DV + 63) / 64;
    int ev, e, cnt;
    float rv[R];
    float col[LEVEL_SEG][CPL];
};

template <typename T, int R, int DV, bool KEYCOLS, bool QUERYCOLS>
__device__ __forceinline__ void seg_load(const PathArgs& a, const LvRow& rw, const int32_t* E,
                                         int ml, int beg, int lane, SegData<T, R, DV>& S) {
    constexpr int CPL = SegData<T, R, DV>::CPL;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    S.cnt = ml - beg < LEVEL_SEG ? ml - beg : LEVEL_SEG;
    const bool in = lane < S.cnt;
    S.ev = in ? E[beg + lane] : 0;
    S.e = lv_e(S.ev);
    const long row = rw.row0 + (long)(S.e >> 1) * a.H;
    if (in) load_row<T, R>(((S.e & 1) ? sq : sk) + row * R, S.rv);
    else
#pragma unroll
        for (int r = 0; r < R; ++r) S.rv[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < LEVEL_SEG; ++t) {
        const int et = rl(S.e, t);
        const bool isq = et & 1;
        const bool need = t < S.cnt && (isq ? QUERYCOLS : KEYCOLS);
        const long rt = rw.row0 + (long)(et >> 1) * a.H;
        const T* src = (isq ? dout : v) + rt * DV;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int cl = lane + 64 * c;
            S.col[t][c] = (need && cl < DV) ? elem<T>(src + cl) : 0.0f;
        }
    }
}

// c_l of a query (lse2 l2) at level l: p_l - p_{l-1}
__device__ __forceinline__ float level_c(const float* lut, int l, float l2) {
    const float p = exp2_fp32(lut[l] - l2);
    return l > 1 ? p - exp2_fp32(lut[l - 1] - l2) : p - 0.0f;
}

// the wave's (level row, segment of any level) of a grid (B*H, ceil(level_segs / LV_WAVES)):
// false when there is none
struct SegPos {
    int bh, l, s, g, o0, ml;
};
__device__ __forceinline__ bool seg_pos(const PathArgs& a, SegPos& P, LvRow& rw) {
    const int BH = a.B * a.H;
    if ((int)blockIdx.x >= a.o.dcount[2]) return false;
    P.bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + blockIdx.x]);
    if (!a.hard[P.bh]) return false;
    rw = lv_row(a, P.bh);
    const int nlev = rw.meta[0];
    P.g = (int)blockIdx.y * LV_WAVES + wave_id();
    if (P.g >= rw.segbase(nlev)) return false;
    int l = 1;
    while (rw.segbase(l) <= P.g) ++l;
    P.l = l;
    P.s = P.g - rw.segbase(l - 1);
    P.o0 = rw.off(l - 1);
    P.ml = rw.off(l) - P.o0;
    return true;
}

// ---------------------------------------------------------------------------------------
// Segment totals: wave per segment.  Forward (KEYS false): the keys of the segment's last
// piece when its group continues into the next segment (T_s, layout [r][d], in lvP); key
// side: the queries of its first piece, descending, when its group began in an earlier
// segment (U_s, [d][r], in lvQ).  Also each segment's flags (lvF / lvFk).
template <typename T, int R, int DV, bool KEYS>
__global__ __launch_bounds__(LV_THREADS) void level_tot_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, RD = R * DV;
    SegPos P;
    LvRow rw;
    if (!seg_pos(a, P, rw)) return;
    const int lane = lane_id(), beg = P.s * LEVEL_SEG;
    const int32_t* E = rw.list(P.l);
    const long sb = (long)P.bh * level_segs(a.n) + P.g;
    SegData<T, R, DV> S;
    seg_load<T, R, DV, !KEYS, KEYS>(a, rw, E, P.ml, beg, lane, S);
    const unsigned long long st = __ballot(lane < S.cnt && (S.ev & LEVEL_START));
    if (lane == 0) (KEYS ? a.o.lvFk : a.o.lvF)[sb] = (uint8_t)((st ? 1 : 0) | ((st & 1ull) ? 2 : 0));
    float acc[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[r][c] = 0.0f;
    if constexpr (!KEYS) {
        if (beg + LEVEL_SEG >= P.ml || (E[beg + LEVEL_SEG] & LEVEL_START)) return;
        const int ls = st ? 63 - __clzll((long long)st) : 0;
#pragma unroll
        for (int t = 0; t < LEVEL_SEG; ++t) {
            if (t >= ls && !(rl(S.e, t) & 1)) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float x = rlf(S.rv[r], t);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) acc[r][c] = __builtin_fmaf(x, S.col[t][c], acc[r][c]);
                }
            }
        }
    } else {
        if (P.s == 0 || (st & 1ull)) return;
        const unsigned long long after = st & ~1ull;
        const int fe = after ? __builtin_ctzll(after) : S.cnt;
        const float* lut = a.lut + (long)rw.h * a.lut_stride;
        float ar[R];
        {
            const bool isq = lane < S.cnt && (S.e & 1);
            const float c = isq ? level_c(lut, P.l, a.lse2[rw.so + (S.e >> 1)]) : 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) ar[r] = c * S.rv[r];
        }
#pragma unroll
        for (int t = LEVEL_SEG - 1; t >= 0; --t) {
            if (t < fe && (rl(S.e, t) & 1)) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float x = rlf(ar[r], t);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) acc[r][c] = __builtin_fmaf(x, S.col[t][c], acc[r][c]);
                }
            }
        }
    }
    float* tot = KEYS ? a.o.lvQ : a.o.lvP;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int col = lane + 64 * c;
        if (col < DV)
#pragma unroll
            for (int r = 0; r < R; ++r)
                tot[sb * RD + (KEYS ? col * R + r : r * DV + col)] = acc[r][c];
    }
}

// ---------------------------------------------------------------------------------------
// The prefix of segment s (wave-uniform; forward / query side, KEYS false): the group of its
// first entry began in segment s0 < s; P_s = ((T_{s0} + T_{s0+1}) + ...) + T_{s-1} over the
// totals of the segments in between (each wholly inside the group).  Key side: the group of
// the last entry runs on to segment s1 > s; Q_s = ((U_{s1} + U_{s1-1}) + ...) + U_{s+1}.
// Flags: bit 0 a group starts in the segment, bit 1 at its first entry.
template <int R, int DV, bool KEYS>
__device__ __forceinline__ void seg_prefix(const float* tot, const uint8_t* fl, long sb0,
                                           int s, int nseg, int lane,
                                           float (&run)[R][(DV + 63) / 64]) {
    constexpr int CPL = (DV + 63) / 64, RD = R * DV;
    // the chain's far end
    int t0;
    if constexpr (!KEYS) {
        t0 = -1;
        for (int w0 = s - 1; t0 < 0; w0 -= 64) {  // segment 0 always holds a start
            const int t = w0 - lane;
            const unsigned long long hit = __ballot(t >= 0 && (fl[sb0 + t] & 1));
            if (hit) t0 = w0 - __builtin_ctzll(hit);
        }
    } else {
        t0 = -1;
        for (int w0 = s + 1; t0 < 0; w0 += 64) {
            const int t = w0 + lane;
            // t ends the chain unless it holds no start and its group runs into t + 1
            const bool end = t < nseg &&
                             ((fl[sb0 + t] & 1) || t + 1 >= nseg || (fl[sb0 + t + 1] & 2));
            const unsigned long long hit = __ballot(end);
            if (hit) t0 = w0 + __builtin_ctzll(hit);
        }
    }
    auto load = [&](int t, float (&x)[R][CPL]) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
#pragma unroll
            for (int r = 0; r < R; ++r)
                x[r][c] = col < DV ? tot[(sb0 + t) * RD + (KEYS ? col * R + r : r * DV + col)]
                                   : 0.0f;
        }
    };
    load(t0, run);
    const int len = KEYS ? t0 - s - 1 : s - 1 - t0;  // further totals to add
    for (int k0 = 0; k0 < len; k0 += 8) {
        float x[8][R][CPL];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (k0 + u < len) load(KEYS ? t0 - 1 - k0 - u : t0 + 1 + k0 + u, x[u]);
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (k0 + u < len)
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int c = 0; c < CPL; ++c) run[r][c] = run[r][c] + x[u][r][c];
    }
}

// ---------------------------------------------------------------------------------------
// Segment walks: wave per (level row, segment of any level).  MODE 0: forward y_l per query
// entry; 1: backward z_l per query entry; 2: backward dv_l, dk_l per key entry (descending).
// Each also records its entries' list indices (lvqidx for modes 0 and 1, lvkidx for 2).
template <typename T, int R, int DV, int MODE>
__global__ __launch_bounds__(LV_THREADS) void level_scan_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, RD = R * DV;
    SegPos P;
    LvRow rw;
    if (!seg_pos(a, P, rw)) return;
    const int lane = lane_id(), n = a.n, beg = P.s * LEVEL_SEG, l = P.l;
    const int32_t* E = rw.list(P.l);
    const long sb = (long)P.bh * level_segs(n) + P.g;
    const long eb = rw.ebase + P.o0 + beg;  // per-entry buffer slot of entry 0
    SegData<T, R, DV> S;
    seg_load<T, R, DV, true, MODE != 0>(a, rw, E, P.ml, beg, lane, S);
    if (lane < S.cnt && (S.e & 1) == (MODE == 2 ? 0 : 1))
        (MODE == 2 ? a.o.lvkidx : a.o.lvqidx)[(long)P.bh * LEVEL_MAX * n + (long)(l - 1) * n +
                                             (S.e >> 1)] = (uint16_t)(beg + lane);
    float M[R][CPL];
    const int nseg = (P.ml + LEVEL_SEG - 1) / LEVEL_SEG;
    const long sb0 = sb - P.s;  // the level's first segment
    if constexpr (MODE != 2) {
        const bool cont = !(rl(S.ev, 0) & LEVEL_START);
        if (cont) {
            seg_prefix<R, DV, false>(a.o.lvP, a.o.lvF, sb0, P.s, nseg, lane, M);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) M[r][c] = 0.0f;
        }
#pragma unroll
        for (int t = 0; t < LEVEL_SEG; ++t) {
            if (t < S.cnt) {
                const int ev = rl(S.ev, t);
                if (t > 0 && (ev & LEVEL_START))
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int c = 0; c < CPL; ++c) M[r][c] = 0.0f;
                if (!(ev & 1)) {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float x = rlf(S.rv[r], t);
#pragma unroll
                        for (int c = 0; c < CPL; ++c)
                            M[r][c] = __builtin_fmaf(x, S.col[t][c], M[r][c]);
                    }
                } else if constexpr (MODE == 0) {
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        float y = 0.0f;
#pragma unroll
                        for (int r = 0; r < R; ++r) y = __builtin_fmaf(rlf(S.rv[r], t), M[r][c], y);
                        const int col = lane + 64 * c;
                        if (col < DV) a.o.lvY[(eb + t) * DV + col] = y;
                    }
                } else {
                    float z[R];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float p = lane < DV ? S.col[t][0] * M[r][0] : 0.0f;
                        if (CPL > 1 && lane + 64 < DV)
                            p = __builtin_fmaf(S.col[t][CPL - 1], M[r][CPL - 1], p);
                        z[r] = lane_tree(p);
                    }
                    if (lane == 0) store_f32_row_l<R>(a.o.lvZ + (eb + t) * R, z);
                }
            }
        }
    } else {
        const float* lut = a.lut + (long)rw.h * a.lut_stride;
        float ar[R];
        {
            const bool isq = lane < S.cnt && (S.e & 1);
            const float c = isq ? level_c(lut, l, a.lse2[rw.so + (S.e >> 1)]) : 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) ar[r] = c * S.rv[r];
        }
        const bool cont = beg + LEVEL_SEG < P.ml && !(E[beg + LEVEL_SEG] & LEVEL_START);
        if (cont) {
            seg_prefix<R, DV, true>(a.o.lvQ, a.o.lvFk, sb0, P.s, nseg, lane, M);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) M[r][c] = 0.0f;
        }
#pragma unroll
        for (int t = LEVEL_SEG - 1; t >= 0; --t) {
            if (t < S.cnt) {
                if (t + 1 < S.cnt && (rl(S.ev, t + 1) & LEVEL_START))
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int c = 0; c < CPL; ++c) M[r][c] = 0.0f;
                const int ev = rl(S.ev, t);
                if (ev & 1) {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float x = rlf(ar[r], t);
#pragma unroll
                        for (int c = 0; c < CPL; ++c)
                            M[r][c] = __builtin_fmaf(x, S.col[t][c], M[r][c]);
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        float y = 0.0f;
#pragma unroll
                        for (int r = 0; r < R; ++r) y = __builtin_fmaf(rlf(S.rv[r], t), M[r][c], y);
                        const int col = lane + 64 * c;
                        if (col < DV) a.o.lvY[(eb + t) * DV + col] = y;
                    }
                    float dk[R];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float p = lane < DV ? S.col[t][0] * M[r][0] : 0.0f;
                        if (CPL > 1 && lane + 64 < DV)
                            p = __builtin_fmaf(S.col[t][CPL - 1], M[r][CPL - 1], p);
                        dk[r] = lane_tree(p);
                    }
                    if (lane == 0) store_f32_row_l<R>(a.o.lvK + (eb + t) * R, dk);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// Combines: wave per query (key), lanes = columns for the DV-wide sums; lane l - 1 fetches
// level l's list index, entry (count) and per-entry slot, so the levels' loads are in flight
// together.  The level sums themselves run in ascending level order.
struct LevelSlots {
    long ei;   // lane l - 1: per-entry slot of the position's level-l entry
    int cnt;   // its key count (queries)
};
__device__ __forceinline__ LevelSlots level_slots(const PathArgs& a, const LvRow& rw,
                                                  const uint16_t* idx, int pos, int levels,
                                                  int lane) {
    LevelSlots s{0, 0};
    if (lane < levels) {
        const int o = rw.off(lane);
        const int x = idx[(long)lane * rw.n + pos];
        s.ei = rw.ebase + o + x;
        s.cnt = lv_n(rw.list(lane + 1)[x]);
    }
    return s;
}

template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_fcombine_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64;
    const int BH = a.B * a.H, n = a.n, lane = lane_id();
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const long nw = (long)gridDim.x * LV_WAVES;
    for (long x = (long)blockIdx.x * LV_WAVES + wave_id(); x < items; x += nw) {
        const int bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + (int)(x / n)]);
        const int i = (int)(x % n);
        if (!a.hard[bh]) continue;
        const LvRow rw = lv_row(a, bh);
        const int4 info = a.o.lvq[rw.so + i];
        const int Lq = __builtin_amdgcn_readfirstlane(info.x);
        const float* lut = a.lut + (long)rw.h * a.lut_stride;
        const LevelSlots ls =
            level_slots(a, rw, a.o.lvqidx + (long)bh * LEVEL_MAX * n, i, Lq, lane);
        // m: the largest LUT[l] over the lengths present (n_l > n_{l+1}), at least 0
        const int nnext = __shfl_down(ls.cnt, 1);
        const bool present = lane < Lq && ls.cnt > (lane + 1 < Lq ? nnext : 0);
        float m = (present && lut[lane + 1] > 0.0f) ? lut[lane + 1] : 0.0f;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, o));
        const float pl = lane < Lq ? exp2_fp32(lut[lane + 1] - m) : 0.0f;
        const float pprev = __shfl_up(pl, 1);
        const float cl = pl - (lane > 0 ? pprev : 0.0f);
        float den = exp2_fp32(-m), acc[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[c] = 0.0f;
        for (int l0 = 0; l0 < Lq; l0 += 8) {
            float y[8][CPL];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (l0 + u < Lq) {
                    const long ei = (long)rl((int)ls.ei, l0 + u) |
                                    ((long)rl((int)(ls.ei >> 32), l0 + u) << 32);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const int col = lane + 64 * c;
                        y[u][c] = col < DV ? a.o.lvY[ei * DV + col] : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (l0 + u < Lq) {
                    const float c = rlf(cl, l0 + u);
                    den = __builtin_fmaf(c, (float)rl(ls.cnt, l0 + u), den);
#pragma unroll
                    for (int cc = 0; cc < CPL; ++cc) acc[cc] = __builtin_fmaf(c, y[u][cc], acc[cc]);
                }
            }
        }
        const long orow = (rw.row0 + (long)i * a.H) * DV;
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) {
            const int col = lane + 64 * cc;
            if (col < DV) {
                const float o = acc[cc] / den;
                if (a.out_dtype == DTYPE_F32)
                    reinterpret_cast<float*>(a.out)[orow + col] = o;
                else
                    reinterpret_cast<uint16_t*>(a.out)[orow + col] = (uint16_t)f32_to_bf16_bits(o);
            }
        }
        if (lane == 0) {
            a.lse2[rw.so + i] = m + log2_fp32(den);
            if (a.lmax) a.lmax[rw.so + i] = Lq;
            if (a.jarg) a.jarg[rw.so + i] = Lq > 0 ? info.y : -1;
        }
    }
}

// backward rows combine: wave per query; lane l - 1 holds level l's z_l
template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_rcombine_kernel(PathArgs a) {
    const int BH = a.B * a.H, n = a.n, lane = lane_id();
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const long nw = (long)gridDim.x * LV_WAVES;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    for (long x = (long)blockIdx.x * LV_WAVES + wave_id(); x < items; x += nw) {
        const int bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + (int)(x / n)]);
        const int i = (int)(x % n);
        if (!a.hard[bh]) continue;
        const LvRow rw = lv_row(a, bh);
        const int Lq = __builtin_amdgcn_readfirstlane(a.o.lvq[rw.so + i].x);
        const float* lut = a.lut + (long)rw.h * a.lut_stride;
        const float* glut = a.dlut + (long)rw.h * a.lut_stride;
        const long qrow = rw.row0 + (long)i * a.H;
        const LevelSlots ls =
            level_slots(a, rw, a.o.lvqidx + (long)bh * LEVEL_MAX * n, i, Lq, lane);
        float zl[R];
        if (lane < Lq) load_row<float, R>(a.o.lvZ + ls.ei * R, zl);
        else
#pragma unroll
            for (int r = 0; r < R; ++r) zl[r] = 0.0f;
        float sqr[R];
        load_row<T, R>(sq + qrow * R, sqr);
        const float l2 = a.lse2[rw.so + i];
        const float cc = glut[i + 1];
        // per lane (level l = lane + 1): p_l, c_l, F_l, dF_l, w_l
        const float pl = lane < Lq ? exp2_fp32(lut[lane + 1] - l2) : 0.0f;
        const float Fl = lane < Lq ? pl * (glut[lane + 1] - cc) : 0.0f;
        const float pp = __shfl_up(pl, 1), fp = __shfl_up(Fl, 1);
        const float cl = pl - (lane > 0 ? pp : 0.0f);
        const float dF = Fl - (lane > 0 ? fp : 0.0f);
        float wl = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) wl = __builtin_fmaf(sqr[r], zl[r], wl);
        float u = 0.0f, vv = 0.0f, ww = 0.0f, z = 0.0f, dq[R];
#pragma unroll
        for (int r = 0; r < R; ++r) dq[r] = 0.0f;
        for (int l = 0; l < Lq; ++l) {
            const float c = rlf(cl, l), d = rlf(dF, l), w = rlf(wl, l);
            const float fn = (float)rl(ls.cnt, l);
#pragma unroll
            for (int r = 0; r < R; ++r) dq[r] = __builtin_fmaf(c, rlf(zl[r], l), dq[r]);
            u = __builtin_fmaf(c, w, u);
            vv = __builtin_fmaf(d, fn, vv);
            ww = __builtin_fmaf(d, w, ww);
            z = __builtin_fmaf(c, fn, z);
        }
        if (lane == 0) {
            store_f32_row_l<R>(a.dsq + qrow * R, dq);
            const float f = exp2_fp32(-l2);
            const float mass = z + f;
            const float mean = __builtin_fmaf(-f, cc, vv) / mass;
            a.rowtau[rw.so + i] = __builtin_fmaf(-u, mean, ww) / mass;
        }
    }
}

// backward keys combine: wave per key (lanes = columns)
template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_kcombine_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64;
    const int BH = a.B * a.H, n = a.n, lane = lane_id();
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const long nw = (long)gridDim.x * LV_WAVES;
    for (long x = (long)blockIdx.x * LV_WAVES + wave_id(); x < items; x += nw) {
        const int bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + (int)(x / n)]);
        const int j = (int)(x % n);
        if (!a.hard[bh]) continue;
        const LvRow rw = lv_row(a, bh);
        const int Kk = __builtin_amdgcn_readfirstlane(a.o.lvq[rw.so + j].w);
        long ei = 0;
        if (lane < Kk)
            ei = rw.ebase + rw.off(lane) + a.o.lvkidx[(long)bh * LEVEL_MAX * n + (long)lane * n + j];
        float dkl[R];
        if (lane < Kk) load_row<float, R>(a.o.lvK + ei * R, dkl);
        else
#pragma unroll
            for (int r = 0; r < R; ++r) dkl[r] = 0.0f;
        float dvv[CPL], dk[R];
#pragma unroll
        for (int c = 0; c < CPL; ++c) dvv[c] = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) dk[r] = 0.0f;
        for (int l0 = 0; l0 < Kk; l0 += 8) {
            float y[8][CPL];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (l0 + u < Kk) {
                    const long e2 = (long)rl((int)ei, l0 + u) | ((long)rl((int)(ei >> 32), l0 + u) << 32);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const int col = lane + 64 * c;
                        y[u][c] = col < DV ? a.o.lvY[e2 * DV + col] : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int l = l0 + u;
                if (l < Kk) {
#pragma unroll
                    for (int c = 0; c < CPL; ++c) dvv[c] = l == 0 ? y[u][c] : dvv[c] + y[u][c];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float d = rlf(dkl[r], l);
                        dk[r] = l == 0 ? d : dk[r] + d;
                    }
                }
            }
        }
        const long krow = rw.row0 + (long)j * a.H;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
            if (col < DV) a.dv[krow * DV + col] = dvv[c];
        }
        if (lane == 0) store_f32_row_l<R>(a.dsk + krow * R, dk);
    }
}

// ---------------------------------------------------------------------------------------
// launchers: (R, DV) pairs with R * DV <= LEVEL_RDV (other shapes never have level rows)
template <typename T, int R, int DV>
static hipError_t level_go(const PathArgs& a, int which, hipStream_t s) {
    const unsigned BH = (unsigned)(a.B * a.H);
    const dim3 wg(BH, (unsigned)((level_segs(a.n) + LV_WAVES - 1) / LV_WAVES));
    if (which == 0 || which == 1)
        hipLaunchKernelGGL((level_tot_kernel<T, R, DV, false>), wg, dim3(LV_THREADS), 0, s, a);
    else
        hipLaunchKernelGGL((level_tot_kernel<T, R, DV, true>), wg, dim3(LV_THREADS), 0, s, a);
    if (which == 0) {
        hipLaunchKernelGGL((level_scan_kernel<T, R, DV, 0>), wg, dim3(LV_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_fcombine_kernel<T, R, DV>), dim3(LV_GRID), dim3(LV_THREADS), 0,
                           s, a);
    } else if (which == 1) {
        hipLaunchKernelGGL((level_scan_kernel<T, R, DV, 1>), wg, dim3(LV_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_rcombine_kernel<T, R, DV>), dim3(LV_GRID), dim3(LV_THREADS), 0,
                           s, a);
    } else {
        hipLaunchKernelGGL((level_scan_kernel<T, R, DV, 2>), wg, dim3(LV_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_kcombine_kernel<T, R, DV>), dim3(LV_GRID), dim3(LV_THREADS), 0,
                           s, a);
    }
    return hipGetLastError();
}

template <typename T>
static hipError_t level_dispatch(const PathArgs& a, int R, int DV, int which, hipStream_t s) {
#define LV_CASE(RR, DD) \
    if (R == RR && DV == DD) return level_go<T, RR, DD>(a, which, s);
    LV_CASE(2, 32) LV_CASE(2, 64) LV_CASE(2, 128)
    LV_CASE(4, 32) LV_CASE(4, 64) LV_CASE(4, 128)
    LV_CASE(8, 32) LV_CASE(8, 64)
    LV_CASE(16, 32)
#undef LV_CASE
    return hipSuccess;  // no level rows at other shapes
}

static hipError_t level_launch(const PathArgs& a, int R, int DV, int dtype, int which,
                               hipStream_t s) {
    if (!a.o.lvent || a.dstart || a.wlo || a.n > LEVEL_MAX_N || R * DV > LEVEL_RDV)
        return hipSuccess;
    if (dtype == DTYPE_BF16) return level_dispatch<bf16_t>(a, R, DV, which, s);
    if (dtype == DTYPE_F32) return level_dispatch<float>(a, R, DV, which, s);
    return hipErrorInvalidValue;
}

hipError_t launch_level_forward(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {
    return level_launch(a, R, DV, dtype, 0, s);
}
hipError_t launch_level_rows(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {
    return level_launch(a, R, DV, dtype, 1, s);
}
hipError_t launch_level_keys(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {
    return level_launch(a, R, DV, dtype, 2, s);
}

}  // namespace dism
