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
// Level lists are cut into segments of LEVEL_SEG entries.  level_seg_kernel forms, per
// segment whose last group piece continues into the next segment, that piece's key sum T_s,
// then per group the prefixes P (P_{s+1} = P_s + T_s, P_{s+1} = T_s where the group began in
// segment s).  level_scan_kernel then walks every segment with one wave: M starts from the
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

namespace dism {

constexpr int LV_SEG_THREADS = 1024;  // level_seg_kernel: one workgroup per (row, level)
constexpr int LV_THREADS = 256;
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

// per-row views of the level state
struct LvRow {
    const int32_t* ent;   // the row's kept entries, all levels
    const int32_t* meta;
    const uint16_t* qidx;
    const uint16_t* kidx;
    const uint16_t* cnt;
    int bh, b, h, n;
    long so, row0, ebase;  // ebase: the row's first entry slot (per-entry buffers)
    __device__ int off(int l) const { return meta[1 + l]; }           // level l+1 begins
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
    r.ent = a.o.lvent + r.ebase;
    r.meta = a.o.lvmeta + (long)bh * LEVEL_META;
    r.qidx = a.o.lvqidx + (long)bh * LEVEL_MAX * n;
    r.kidx = a.o.lvkidx + (long)bh * LEVEL_MAX * n;
    r.cnt = a.o.lvcnt + (long)bh * LEVEL_MAX * n;
    return r;
}

// One segment of a level list held by a wave: lane t < cnt holds entry t (ev with its
// group-start flag, e without), its row (sk of a key, sq of a query) in rv, and for each
// entry t every lane holds column lane + 64 c of its value row (keys) or gradient row
// (queries), as `need` selects, in col[t][c].
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
    S.e = S.ev & ~LEVEL_START;
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

// c_l of query position p (lse2 l2), level l: p_l - p_{l-1}
__device__ __forceinline__ float level_c(const float* lut, int l, float l2) {
    const float p = exp2_fp32(lut[l] - l2);
    return l > 1 ? p - exp2_fp32(lut[l - 1] - l2) : p - 0.0f;
}

// ---------------------------------------------------------------------------------------
// Segment totals and prefixes of one (level row, level): forward T / P over keys (KEYS
// false), or the key side's U / Q over queries (KEYS true).  Grid (B*H, LEVEL_MAX).
template <typename T, int R, int DV, bool KEYS>
__global__ __launch_bounds__(LV_SEG_THREADS) void level_seg_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, RD = R * DV;
    constexpr int NW = LV_SEG_THREADS / 64;
    __shared__ uint8_t s_any[LV_MAX_SEGS], s_first[LV_MAX_SEGS];
    const int BH = a.B * a.H;
    if ((int)blockIdx.x >= a.o.dcount[2]) return;
    const int bh = a.o.dlist[2 * BH + blockIdx.x];
    const int l = (int)blockIdx.y + 1;
    if (!a.hard[bh]) return;
    const LvRow rw = lv_row(a, bh);
    if (l > rw.meta[0]) return;
    const int lane = lane_id(), w = wave_id();
    const int o0 = rw.off(l - 1), ml = rw.off(l) - o0;
    const int nseg = (ml + LEVEL_SEG - 1) / LEVEL_SEG;
    const int32_t* E = rw.ent + o0;
    const long sbase = (long)bh * level_segs(a.n) + rw.segbase(l - 1);
    // one buffer per direction: the totals, each overwritten by the prefix it produces once
    // read (P_{s+1} into T_s's slot, Q_{s-1} into U_s's slot)
    float* tot = KEYS ? a.o.lvQ : a.o.lvP;
    float* pre = tot;
    const float* lut = a.lut + (long)rw.h * a.lut_stride;
    auto ix = [&](int seg, int r, int col) {
        return (sbase + seg) * RD + (KEYS ? col * R + r : r * DV + col);
    };
    // ---- phase 1: segment flags; totals of the pieces that cross a segment boundary
    for (int s = w; s < nseg; s += NW) {
        const int beg = s * LEVEL_SEG;
        SegData<T, R, DV> S;
        seg_load<T, R, DV, !KEYS, KEYS>(a, rw, E, ml, beg, lane, S);
        const unsigned long long st = __ballot(lane < S.cnt && (S.ev & LEVEL_START));
        if (lane == 0) {
            s_any[s] = st != 0ull;
            s_first[s] = st & 1ull;
        }
        float acc[R][CPL];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) acc[r][c] = 0.0f;
        if constexpr (!KEYS) {
            // the last piece of s, when its group continues into s + 1
            if (s + 1 >= nseg || (E[beg + LEVEL_SEG] & LEVEL_START)) continue;
            const int ls = st ? 63 - __clzll((long long)st) : 0;
#pragma unroll
            for (int t = 0; t < LEVEL_SEG; ++t) {
                if (t >= ls && !(rl(S.e, t) & 1)) {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float x = rlf(S.rv[r], t);
#pragma unroll
                        for (int c = 0; c < CPL; ++c)
                            acc[r][c] = __builtin_fmaf(x, S.col[t][c], acc[r][c]);
                    }
                }
            }
        } else {
            // the first piece of s, when its group began in an earlier segment
            if (s == 0 || (st & 1ull)) continue;
            const unsigned long long after = st & ~1ull;
            const int fe = after ? __builtin_ctzll(after) : S.cnt;
            float ar[R];
            {
                const bool isq = lane < S.cnt && (S.e & 1);
                const float c = isq ? level_c(lut, l, a.lse2[rw.so + (S.e >> 1)]) : 0.0f;
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
                        for (int c = 0; c < CPL; ++c)
                            acc[r][c] = __builtin_fmaf(x, S.col[t][c], acc[r][c]);
                    }
                }
            }
        }
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
            if (col < DV)
#pragma unroll
                for (int r = 0; r < R; ++r) tot[ix(s, r, col)] = acc[r][c];
        }
    }
    __syncthreads();
    // ---- phase 2: one wave per chain of segments crossed by one group
    for (int s = w; s < nseg; s += NW) {
        float run[R][CPL];
        auto load_tot = [&](int seg, float (&x)[R][CPL]) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
#pragma unroll
                for (int r = 0; r < R; ++r) x[r][c] = col < DV ? tot[ix(seg, r, col)] : 0.0f;
            }
        };
        auto store_pre = [&](int seg) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                if (col < DV)
#pragma unroll
                    for (int r = 0; r < R; ++r) pre[ix(seg, r, col)] = run[r][c];
            }
        };
        if constexpr (!KEYS) {
            // head: s holds a start and its last piece continues into s + 1; the chain runs
            // on through the segments that hold no start
            if (s + 1 >= nseg || s_first[s + 1] || !s_any[s]) continue;
            int t1 = s + 1;
            while (t1 + 1 < nseg && !s_first[t1 + 1] && !s_any[t1]) ++t1;
            load_tot(s, run);
            store_pre(s);  // P_{s+1}
            for (int t = s + 1; t < t1; t += 4) {
                float x[4][R][CPL];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (t + u < t1) load_tot(t + u, x[u]);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (t + u < t1) {
#pragma unroll
                        for (int r = 0; r < R; ++r)
#pragma unroll
                            for (int c = 0; c < CPL; ++c) run[r][c] = run[r][c] + x[u][r][c];
                        store_pre(t + u);  // P_{t+u+1}
                    }
            }
        } else {
            // head: s's first piece continues from s - 1 and does not run through all of s
            // into s + 1; the chain runs down through the segments that hold no start
            if (s == 0 || s_first[s]) continue;
            if (!s_any[s] && s + 1 < nseg && !s_first[s + 1]) continue;
            int t1 = s - 1;
            while (t1 >= 1 && !s_any[t1]) --t1;
            load_tot(s, run);
            store_pre(s);  // Q_{s-1}
            for (int t = s - 1; t > t1; t -= 4) {
                float x[4][R][CPL];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (t - u > t1) load_tot(t - u, x[u]);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (t - u > t1) {
#pragma unroll
                        for (int r = 0; r < R; ++r)
#pragma unroll
                            for (int c = 0; c < CPL; ++c) run[r][c] = run[r][c] + x[u][r][c];
                        store_pre(t - u);  // Q_{t-u-1}
                    }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// Segment walks: wave per (level row, segment of any level).  MODE 0: forward y_l per query
// entry; 1: backward z_l per query entry; 2: backward dv_l, dk_l per key entry (descending).
// Grid (B*H, ceil(level_segs(N) / 4)).
template <typename T, int R, int DV, int MODE>
__global__ __launch_bounds__(LV_THREADS) void level_scan_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, RD = R * DV;
    const int BH = a.B * a.H;
    if ((int)blockIdx.x >= a.o.dcount[2]) return;
    const int bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + blockIdx.x]);
    if (!a.hard[bh]) return;
    const LvRow rw = lv_row(a, bh);
    const int nlev = rw.meta[0];
    const int g = (int)blockIdx.y * (LV_THREADS / 64) + wave_id();
    if (g >= rw.segbase(nlev)) return;
    int l = 1;
    while (rw.segbase(l) <= g) ++l;
    const int lane = lane_id();
    const int o0 = rw.off(l - 1), ml = rw.off(l) - o0;
    const int s = g - rw.segbase(l - 1), beg = s * LEVEL_SEG;
    const int32_t* E = rw.ent + o0;
    const long sb = (long)bh * level_segs(a.n) + g;
    const long eb = rw.ebase + o0 + beg;  // per-entry buffer slot of entry 0
    SegData<T, R, DV> S;
    seg_load<T, R, DV, true, MODE != 0>(a, rw, E, ml, beg, lane, S);
    float M[R][CPL];
    if constexpr (MODE != 2) {
        const bool cont = !(rl(S.ev, 0) & LEVEL_START);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
#pragma unroll
            for (int r = 0; r < R; ++r)
                M[r][c] = (cont && col < DV) ? a.o.lvP[(sb - 1) * RD + r * DV + col] : 0.0f;
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
                    if (lane == 0)
#pragma unroll
                        for (int r = 0; r < R; ++r) a.o.lvZ[(eb + t) * R + r] = z[r];
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
        const bool cont = beg + LEVEL_SEG < ml && !(E[beg + LEVEL_SEG] & LEVEL_START);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
#pragma unroll
            for (int r = 0; r < R; ++r)
                M[r][c] = (cont && col < DV) ? a.o.lvQ[(sb + 1) * RD + col * R + r] : 0.0f;
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
                    if (lane == 0)
#pragma unroll
                        for (int r = 0; r < R; ++r) a.o.lvK[(eb + t) * R + r] = dk[r];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// forward combine: wave per query (lanes = columns)
template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_fcombine_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64;
    const int BH = a.B * a.H, n = a.n, lane = lane_id();
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const long nw = (long)gridDim.x * (LV_THREADS / 64);
    for (long x = (long)blockIdx.x * (LV_THREADS / 64) + wave_id(); x < items; x += nw) {
        const int bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + (int)(x / n)]);
        const int i = (int)(x % n);
        if (!a.hard[bh]) continue;
        const LvRow rw = lv_row(a, bh);
        const int4 info = a.o.lvq[rw.so + i];
        const int Lq = __builtin_amdgcn_readfirstlane(info.x);
        const float* lut = a.lut + (long)rw.h * a.lut_stride;
        const uint16_t* cn = rw.cnt + i;
        float m = 0.0f;
        for (int l = 1; l <= Lq; ++l) {
            const int n1 = cn[(long)(l - 1) * n];
            const int n2 = l < Lq ? (int)cn[(long)l * n] : 0;
            if (n1 > n2) {
                const float lw = lut[l];
                if (lw > m) m = lw;
            }
        }
        float den = exp2_fp32(-m), pp = 0.0f, acc[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[c] = 0.0f;
        for (int l0 = 1; l0 <= Lq; l0 += 4) {
            float y[4][CPL];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int l = l0 + u;
                if (l <= Lq) {
                    const long ei = rw.ebase + rw.off(l - 1) + rw.qidx[(long)(l - 1) * n + i];
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const int col = lane + 64 * c;
                        y[u][c] = col < DV ? a.o.lvY[ei * DV + col] : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int l = l0 + u;
                if (l <= Lq) {
                    const float p = exp2_fp32(lut[l] - m);
                    const float c = p - pp;
                    pp = p;
                    den = __builtin_fmaf(c, (float)cn[(long)(l - 1) * n], den);
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

// backward rows combine: lane per query
template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_rcombine_kernel(PathArgs a) {
    const int BH = a.B * a.H, n = a.n;
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    for (long x = (long)blockIdx.x * LV_THREADS + threadIdx.x; x < items;
         x += (long)gridDim.x * LV_THREADS) {
        const int bh = a.o.dlist[2 * BH + (int)(x / n)];
        const int i = (int)(x % n);
        if (!a.hard[bh]) continue;
        const LvRow rw = lv_row(a, bh);
        const int Lq = a.o.lvq[rw.so + i].x;
        const float* lut = a.lut + (long)rw.h * a.lut_stride;
        const float* glut = a.dlut + (long)rw.h * a.lut_stride;
        const uint16_t* cn = rw.cnt + i;
        const long qrow = rw.row0 + (long)i * a.H;
        float sqr[R];
        load_row<T, R>(sq + qrow * R, sqr);
        const float l2 = a.lse2[rw.so + i];
        const float cc = glut[i + 1];
        float u = 0.0f, vv = 0.0f, ww = 0.0f, z = 0.0f, pp = 0.0f, fp = 0.0f, dq[R];
#pragma unroll
        for (int r = 0; r < R; ++r) dq[r] = 0.0f;
        for (int l = 1; l <= Lq; ++l) {
            const long ei = rw.ebase + rw.off(l - 1) + rw.qidx[(long)(l - 1) * n + i];
            float zl[R];
            load_row<float, R>(a.o.lvZ + ei * R, zl);
            const float p = exp2_fp32(lut[l] - l2);
            const float c = p - pp;
            const float F = p * (glut[l] - cc);
            const float dF = F - fp;
            pp = p;
            fp = F;
            float wl = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) wl = __builtin_fmaf(sqr[r], zl[r], wl);
            const float fn = (float)cn[(long)(l - 1) * n];
#pragma unroll
            for (int r = 0; r < R; ++r) dq[r] = __builtin_fmaf(c, zl[r], dq[r]);
            u = __builtin_fmaf(c, wl, u);
            vv = __builtin_fmaf(dF, fn, vv);
            ww = __builtin_fmaf(dF, wl, ww);
            z = __builtin_fmaf(c, fn, z);
        }
        store_f32_row_l<R>(a.dsq + qrow * R, dq);
        const float f = exp2_fp32(-l2);
        const float mass = z + f;
        const float mean = __builtin_fmaf(-f, cc, vv) / mass;
        a.rowtau[rw.so + i] = __builtin_fmaf(-u, mean, ww) / mass;
    }
}

// backward keys combine: wave per key (lanes = columns)
template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_kcombine_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64;
    const int BH = a.B * a.H, n = a.n, lane = lane_id();
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const long nw = (long)gridDim.x * (LV_THREADS / 64);
    for (long x = (long)blockIdx.x * (LV_THREADS / 64) + wave_id(); x < items; x += nw) {
        const int bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + (int)(x / n)]);
        const int j = (int)(x % n);
        if (!a.hard[bh]) continue;
        const LvRow rw = lv_row(a, bh);
        const int Kk = __builtin_amdgcn_readfirstlane(a.o.lvq[rw.so + j].w);
        float dvv[CPL], dk[R];
#pragma unroll
        for (int c = 0; c < CPL; ++c) dvv[c] = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) dk[r] = 0.0f;
        for (int l0 = 1; l0 <= Kk; l0 += 4) {
            float y[4][CPL], d[4][R];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int l = l0 + u;
                if (l <= Kk) {
                    const long ei = rw.ebase + rw.off(l - 1) + rw.kidx[(long)(l - 1) * n + j];
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const int col = lane + 64 * c;
                        y[u][c] = col < DV ? a.o.lvY[ei * DV + col] : 0.0f;
                    }
                    load_row<float, R>(a.o.lvK + ei * R, d[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int l = l0 + u;
                if (l <= Kk) {
#pragma unroll
                    for (int c = 0; c < CPL; ++c) dvv[c] = l == 1 ? y[u][c] : dvv[c] + y[u][c];
#pragma unroll
                    for (int r = 0; r < R; ++r) dk[r] = l == 1 ? d[u][r] : dk[r] + d[u][r];
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
    const dim3 sg(BH, LEVEL_MAX);
    const dim3 wg(BH, (unsigned)((level_segs(a.n) + 3) / 4));
    if (which == 0) {
        hipLaunchKernelGGL((level_seg_kernel<T, R, DV, false>), sg, dim3(LV_SEG_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_scan_kernel<T, R, DV, 0>), wg, dim3(LV_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_fcombine_kernel<T, R, DV>), dim3(LV_GRID), dim3(LV_THREADS), 0,
                           s, a);
    } else if (which == 1) {
        hipLaunchKernelGGL((level_seg_kernel<T, R, DV, false>), sg, dim3(LV_SEG_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_scan_kernel<T, R, DV, 1>), wg, dim3(LV_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_rcombine_kernel<T, R, DV>), dim3(LV_GRID / 4), dim3(LV_THREADS),
                           0, s, a);
    } else {
        hipLaunchKernelGGL((level_seg_kernel<T, R, DV, true>), sg, dim3(LV_SEG_THREADS), 0, s, a);
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
