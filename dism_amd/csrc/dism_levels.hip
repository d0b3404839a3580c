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
// segment s).  A query's M starts from its segment's P (when its group began in an earlier
// segment) and adds the keys of its piece before it.  The key side mirrors this (U_s over a
// segment's first piece, Q_{s-1} = Q_s + U_s, queries in descending order).
//
// Waves: one per query (forward, backward rows) or key (backward keys), lanes = value
// columns (DV <= 128: CPL = 1 or 2 per lane); the segment lists are read with one vector
// load and ballots.  Everything is a fixed fp32 sequence, restated by the oracle's
// level_forward_row / level_backward_row (oracle/dism_cpu_model.c):
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

constexpr int LV_THREADS = 256;
constexpr unsigned LV_GRID = 1024;  // persistent workgroups of the per-query / per-key kernels

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

// per-row views of the level state
struct LvRow {
    const int32_t* ent;   // the row's kept entries, all levels
    const int32_t* meta;
    const uint16_t* qidx;
    const uint16_t* kidx;
    const uint16_t* cnt;
    int bh, b, h, n;
    long so, row0;
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
    r.ent = a.o.lvent + (long)bh * LEVEL_BUDGET * n;
    r.meta = a.o.lvmeta + (long)bh * LEVEL_META;
    r.qidx = a.o.lvqidx + (long)bh * LEVEL_MAX * n;
    r.kidx = a.o.lvkidx + (long)bh * LEVEL_MAX * n;
    r.cnt = a.o.lvcnt + (long)bh * LEVEL_MAX * n;
    return r;
}

// M (layout [r][column]) of the query at index x of a level list E (ml entries): from the
// segment prefix Pl (this level's first segment) when its group began in an earlier segment,
// plus its piece's keys before it.
template <typename T, int R, int DV>
__device__ __forceinline__ void query_m(const PathArgs& a, const LvRow& rw, const int32_t* E,
                                        int ml, int x, const float* Pl, int lane,
                                        float (&M)[R][(DV + 63) / 64]) {
    constexpr int CPL = (DV + 63) / 64;
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const int beg = x & ~(LEVEL_SEG - 1), xo = x - beg;
    const int ev = (lane < LEVEL_SEG && beg + lane < ml) ? E[beg + lane] : 0;
    const unsigned long long st = __ballot(lane <= xo && (ev & LEVEL_START));
    unsigned long long km = __ballot(lane < xo && !(ev & 1));
    bool cont = true;
    if (st) {
        const int ps = 63 - __clzll((long long)st);
        km &= ~((1ull << ps) - 1ull);
        cont = false;
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int col = lane + 64 * c;
#pragma unroll
        for (int r = 0; r < R; ++r)
            M[r][c] = (cont && col < DV)
                          ? Pl[(long)(beg / LEVEL_SEG) * (R * DV) + r * DV + col] : 0.0f;
    }
    while (km) {
        const int t = __builtin_ctzll(km);
        km &= km - 1ull;
        const int e = __builtin_amdgcn_readfirstlane(__shfl(ev, t)) & ~LEVEL_START;
        const long krow = rw.row0 + (long)(e >> 1) * a.H;
        float skr[R];
        load_row<T, R>(sk + krow * R, skr);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
            if (col < DV) {
                const float vv = elem<T>(v + krow * DV + col);
#pragma unroll
                for (int r = 0; r < R; ++r) M[r][c] = __builtin_fmaf(skr[r], vv, M[r][c]);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// Segment totals and prefixes of one (level row, level): forward P over keys (KEYS false),
// or the key side's c_l per query entry, U and Q (KEYS true).  Grid (B*H, LEVEL_MAX).
template <typename T, int R, int DV, bool KEYS>
__global__ __launch_bounds__(LV_THREADS) void level_seg_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, RD = R * DV;
    const int BH = a.B * a.H;
    if ((int)blockIdx.x >= a.o.dcount[2]) return;
    const int bh = a.o.dlist[2 * BH + blockIdx.x];
    const int l = (int)blockIdx.y + 1;
    if (!a.hard[bh]) return;
    const LvRow rw = lv_row(a, bh);
    if (l > rw.meta[0]) return;
    const int lane = lane_id(), w = wave_id(), tid = threadIdx.x;
    const int o0 = rw.off(l - 1), ml = rw.off(l) - o0;
    const int nseg = (ml + LEVEL_SEG - 1) / LEVEL_SEG;
    const int32_t* E = rw.ent + o0;
    const long sbase = (long)bh * level_segs(a.n) + rw.segbase(l - 1);
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    float* tot = KEYS ? a.o.lvU : a.o.lvT;
    float* pre = KEYS ? a.o.lvQ : a.o.lvP;
    float* cl = a.o.lvc + (long)bh * LEVEL_BUDGET * a.n + o0;
    const float* lut = a.lut + (long)rw.h * a.lut_stride;
    if constexpr (KEYS) {
        // c_l of every query entry of the level
        for (int t = tid; t < ml; t += LV_THREADS) {
            const int e = E[t] & ~LEVEL_START;
            if (e & 1) {
                const float l2 = a.lse2[rw.so + (e >> 1)];
                const float p = exp2_fp32(lut[l] - l2);
                cl[t] = l > 1 ? p - exp2_fp32(lut[l - 1] - l2) : p - 0.0f;
            }
        }
        __syncthreads();
    }
    // ---- phase 1: totals of the pieces that cross a segment boundary
    for (int s = w; s < nseg; s += LV_THREADS / 64) {
        const int beg = s * LEVEL_SEG;
        const int ev = (lane < LEVEL_SEG && beg + lane < ml) ? E[beg + lane] : 0;
        const unsigned long long st = __ballot(lane < LEVEL_SEG && (ev & LEVEL_START));
        float acc[R][CPL];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < CPL; ++c) acc[r][c] = 0.0f;
        if constexpr (!KEYS) {
            // the last piece of s, when its group continues into s + 1
            if (s + 1 >= nseg || (E[beg + LEVEL_SEG] & LEVEL_START)) continue;
            const int ls = st ? 63 - __clzll((long long)st) : 0;
            unsigned long long km = __ballot(lane >= ls && lane < LEVEL_SEG && !(ev & 1));
            while (km) {
                const int t = __builtin_ctzll(km);
                km &= km - 1ull;
                const int e = __builtin_amdgcn_readfirstlane(__shfl(ev, t)) & ~LEVEL_START;
                const long krow = rw.row0 + (long)(e >> 1) * a.H;
                float skr[R];
                load_row<T, R>(sk + krow * R, skr);
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int col = lane + 64 * c;
                    if (col < DV) {
                        const float vv = elem<T>(v + krow * DV + col);
#pragma unroll
                        for (int r = 0; r < R; ++r)
                            acc[r][c] = __builtin_fmaf(skr[r], vv, acc[r][c]);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                if (col < DV)
#pragma unroll
                    for (int r = 0; r < R; ++r) tot[(sbase + s) * RD + r * DV + col] = acc[r][c];
            }
        } else {
            // the first piece of s, when its group began in an earlier segment
            if (s == 0 || (st & 1ull)) continue;
            const unsigned long long after = st & ~1ull;
            const int fe = after ? __builtin_ctzll(after)
                                 : (ml - beg < LEVEL_SEG ? ml - beg : LEVEL_SEG);
            unsigned long long qm = __ballot(lane < fe && (ev & 1));
            while (qm) {
                const int t = 63 - __clzll((long long)qm);
                qm &= ~(1ull << t);
                const int e = __builtin_amdgcn_readfirstlane(__shfl(ev, t)) & ~LEVEL_START;
                const long qrow = rw.row0 + (long)(e >> 1) * a.H;
                const float c = cl[beg + t];
                float ar[R];
                load_row<T, R>(sq + qrow * R, ar);
#pragma unroll
                for (int r = 0; r < R; ++r) ar[r] = c * ar[r];
#pragma unroll
                for (int cc = 0; cc < CPL; ++cc) {
                    const int col = lane + 64 * cc;
                    if (col < DV) {
                        const float dd = elem<T>(dout + qrow * DV + col);
#pragma unroll
                        for (int r = 0; r < R; ++r)
                            acc[r][cc] = __builtin_fmaf(ar[r], dd, acc[r][cc]);
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                if (col < DV)
#pragma unroll
                    for (int r = 0; r < R; ++r) tot[(sbase + s) * RD + col * R + r] = acc[r][c];
            }
        }
    }
    __syncthreads();
    // ---- phase 2: one wave per chain of segments crossed by one group
    for (int s = w; s < nseg; s += LV_THREADS / 64) {
        const int beg = s * LEVEL_SEG;
        const int ev = (lane < LEVEL_SEG && beg + lane < ml) ? E[beg + lane] : 0;
        const unsigned long long st = __ballot(lane < LEVEL_SEG && (ev & LEVEL_START));
        float run[R][CPL];
        auto add_tot = [&](int seg, bool first) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                if (col < DV)
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const long ix = (sbase + seg) * RD + (KEYS ? col * R + r : r * DV + col);
                        run[r][c] = first ? tot[ix] : run[r][c] + tot[ix];
                    }
            }
        };
        auto store_pre = [&](int seg) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                if (col < DV)
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        pre[(sbase + seg) * RD + (KEYS ? col * R + r : r * DV + col)] = run[r][c];
            }
        };
        // a segment holding no group start (the whole segment in one group)
        auto inside = [&](int seg) {
            const int b2 = seg * LEVEL_SEG;
            const int e2 = (lane < LEVEL_SEG && b2 + lane < ml) ? E[b2 + lane] : 0;
            return __ballot(lane < LEVEL_SEG && (e2 & LEVEL_START)) == 0ull;
        };
        if constexpr (!KEYS) {
            // head: s holds a start and its last piece continues into s + 1
            if (s + 1 >= nseg || (E[beg + LEVEL_SEG] & LEVEL_START) || !st) continue;
            add_tot(s, true);
            int t = s + 1;
            store_pre(t);
            while (t + 1 < nseg && !(E[(t + 1) * LEVEL_SEG] & LEVEL_START) && inside(t)) {
                add_tot(t, false);
                ++t;
                store_pre(t);
            }
        } else {
            // head: s's first piece continues from s - 1, and s's group does not run through
            // all of s into s + 1
            if (s == 0 || (st & 1ull)) continue;
            const bool through = !(st & ~1ull) && beg + LEVEL_SEG < ml &&
                                 !(E[beg + LEVEL_SEG] & LEVEL_START);
            if (through) continue;
            add_tot(s, true);
            int t = s - 1;
            store_pre(t);
            while (t >= 1 && inside(t)) {
                add_tot(t, false);
                --t;
                store_pre(t);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// forward: wave per query of the level rows
template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_forward_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64;
    const int BH = a.B * a.H, n = a.n, lane = lane_id();
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const long nw = (long)gridDim.x * (LV_THREADS / 64);
    const T* sq = reinterpret_cast<const T*>(a.sq);
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
        float sqr[R];
        load_row<T, R>(sq + (rw.row0 + (long)i * a.H) * R, sqr);
        float den = exp2_fp32(-m), pp = 0.0f, acc[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc[c] = 0.0f;
        const float* P = a.o.lvP + (long)bh * level_segs(n) * (R * DV);
        for (int l = 1; l <= Lq; ++l) {
            const float p = exp2_fp32(lut[l] - m);
            const float c = p - pp;
            pp = p;
            den = __builtin_fmaf(c, (float)cn[(long)(l - 1) * n], den);
            const int o0 = rw.off(l - 1);
            float M[R][CPL];
            query_m<T, R, DV>(a, rw, rw.ent + o0, rw.off(l) - o0,
                              rw.qidx[(long)(l - 1) * n + i],
                              P + (long)rw.segbase(l - 1) * (R * DV), lane, M);
#pragma unroll
            for (int cc = 0; cc < CPL; ++cc) {
                float y = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) y = __builtin_fmaf(sqr[r], M[r][cc], y);
                acc[cc] = __builtin_fmaf(c, y, acc[cc]);
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

// ---------------------------------------------------------------------------------------
// backward, query rows (dSQ, rowtau): wave per query
template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_rows_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64;
    const int BH = a.B * a.H, n = a.n, lane = lane_id();
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const long nw = (long)gridDim.x * (LV_THREADS / 64);
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long x = (long)blockIdx.x * (LV_THREADS / 64) + wave_id(); x < items; x += nw) {
        const int bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + (int)(x / n)]);
        const int i = (int)(x % n);
        if (!a.hard[bh]) continue;
        const LvRow rw = lv_row(a, bh);
        const int Lq = __builtin_amdgcn_readfirstlane(a.o.lvq[rw.so + i].x);
        const float* lut = a.lut + (long)rw.h * a.lut_stride;
        const float* glut = a.dlut + (long)rw.h * a.lut_stride;
        const uint16_t* cn = rw.cnt + i;
        const long qrow = rw.row0 + (long)i * a.H;
        float sqr[R], dor[CPL];
        load_row<T, R>(sq + qrow * R, sqr);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
            dor[c] = col < DV ? elem<T>(dout + qrow * DV + col) : 0.0f;
        }
        const float l2 = a.lse2[rw.so + i];
        const float cc = glut[i + 1];
        float u = 0.0f, vv = 0.0f, ww = 0.0f, z = 0.0f, pp = 0.0f, fp = 0.0f, dq[R];
#pragma unroll
        for (int r = 0; r < R; ++r) dq[r] = 0.0f;
        const float* P = a.o.lvP + (long)bh * level_segs(n) * (R * DV);
        for (int l = 1; l <= Lq; ++l) {
            const float p = exp2_fp32(lut[l] - l2);
            const float c = p - pp;
            const float F = p * (glut[l] - cc);
            const float dF = F - fp;
            pp = p;
            fp = F;
            const int o0 = rw.off(l - 1);
            float M[R][CPL];
            query_m<T, R, DV>(a, rw, rw.ent + o0, rw.off(l) - o0,
                              rw.qidx[(long)(l - 1) * n + i],
                              P + (long)rw.segbase(l - 1) * (R * DV), lane, M);
            float zl[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float t = lane < DV ? dor[0] * M[r][0] : 0.0f;
                if (CPL > 1 && lane + 64 < DV) t = __builtin_fmaf(dor[CPL - 1], M[r][CPL - 1], t);
                zl[r] = lane_tree(t);
            }
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
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) a.dsq[qrow * R + r] = dq[r];
            const float f = exp2_fp32(-l2);
            const float mass = z + f;
            const float mean = __builtin_fmaf(-f, cc, vv) / mass;
            a.rowtau[rw.so + i] = __builtin_fmaf(-u, mean, ww) / mass;
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward, keys (dSK, dV): wave per key
template <typename T, int R, int DV>
__global__ __launch_bounds__(LV_THREADS) void level_keys_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64;
    const int BH = a.B * a.H, n = a.n, lane = lane_id();
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[2]);
    const long items = (long)cnt * n;
    const long nw = (long)gridDim.x * (LV_THREADS / 64);
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long x = (long)blockIdx.x * (LV_THREADS / 64) + wave_id(); x < items; x += nw) {
        const int bh = __builtin_amdgcn_readfirstlane(a.o.dlist[2 * BH + (int)(x / n)]);
        const int j = (int)(x % n);
        if (!a.hard[bh]) continue;
        const LvRow rw = lv_row(a, bh);
        const int Kk = __builtin_amdgcn_readfirstlane(a.o.lvq[rw.so + j].w);
        const long krow = rw.row0 + (long)j * a.H;
        float skr[R], vr[CPL], dvv[CPL], dk[R];
        load_row<T, R>(sk + krow * R, skr);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
            vr[c] = col < DV ? elem<T>(v + krow * DV + col) : 0.0f;
            dvv[c] = 0.0f;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) dk[r] = 0.0f;
        const float* Q = a.o.lvQ + (long)bh * level_segs(n) * (R * DV);
        for (int l = 1; l <= Kk; ++l) {
            const int o0 = rw.off(l - 1), ml = rw.off(l) - o0;
            const int32_t* E = rw.ent + o0;
            const float* cl = a.o.lvc + (long)bh * LEVEL_BUDGET * n + o0;
            const int xk = rw.kidx[(long)(l - 1) * n + j];
            const int beg = xk & ~(LEVEL_SEG - 1), xo = xk - beg;
            const int ev = (lane < LEVEL_SEG && beg + lane < ml) ? E[beg + lane] : 0;
            const unsigned long long stm = __ballot(lane > xo && (ev & LEVEL_START));
            const int pe = stm ? __builtin_ctzll(stm)
                               : (ml - beg < LEVEL_SEG ? ml - beg : LEVEL_SEG);
            const bool cont = !stm && beg + LEVEL_SEG < ml && !(E[beg + LEVEL_SEG] & LEVEL_START);
            unsigned long long qm = __ballot(lane > xo && lane < pe && (ev & 1));
            float K[R][CPL];
            const float* Qs = Q + ((long)rw.segbase(l - 1) + beg / LEVEL_SEG) * (R * DV);
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
#pragma unroll
                for (int r = 0; r < R; ++r) K[r][c] = (cont && col < DV) ? Qs[col * R + r] : 0.0f;
            }
            while (qm) {
                const int t = 63 - __clzll((long long)qm);
                qm &= ~(1ull << t);
                const int e = __builtin_amdgcn_readfirstlane(__shfl(ev, t)) & ~LEVEL_START;
                const long qrow = rw.row0 + (long)(e >> 1) * a.H;
                const float c = cl[beg + t];
                float ar[R];
                load_row<T, R>(sq + qrow * R, ar);
#pragma unroll
                for (int r = 0; r < R; ++r) ar[r] = c * ar[r];
#pragma unroll
                for (int cc = 0; cc < CPL; ++cc) {
                    const int col = lane + 64 * cc;
                    if (col < DV) {
                        const float dd = elem<T>(dout + qrow * DV + col);
#pragma unroll
                        for (int r = 0; r < R; ++r) K[r][cc] = __builtin_fmaf(ar[r], dd, K[r][cc]);
                    }
                }
            }
#pragma unroll
            for (int cc = 0; cc < CPL; ++cc) {
                float y = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) y = __builtin_fmaf(skr[r], K[r][cc], y);
                dvv[cc] = l == 1 ? y : dvv[cc] + y;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float t = lane < DV ? vr[0] * K[r][0] : 0.0f;
                if (CPL > 1 && lane + 64 < DV) t = __builtin_fmaf(vr[CPL - 1], K[r][CPL - 1], t);
                const float d = lane_tree(t);
                dk[r] = l == 1 ? d : dk[r] + d;
            }
        }
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int col = lane + 64 * c;
            if (col < DV) a.dv[krow * DV + col] = dvv[c];
        }
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < R; ++r) a.dsk[krow * R + r] = dk[r];
    }
}

// ---------------------------------------------------------------------------------------
// launchers: (R, DV) pairs with R * DV <= LEVEL_RDV (other shapes never have level rows)
template <typename T, int R, int DV>
static hipError_t level_go(const PathArgs& a, int which, hipStream_t s) {
    const dim3 sg((unsigned)(a.B * a.H), LEVEL_MAX);
    if (which == 0) {
        hipLaunchKernelGGL((level_seg_kernel<T, R, DV, false>), sg, dim3(LV_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_forward_kernel<T, R, DV>), dim3(LV_GRID), dim3(LV_THREADS), 0,
                           s, a);
    } else if (which == 1) {
        hipLaunchKernelGGL((level_seg_kernel<T, R, DV, false>), sg, dim3(LV_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_rows_kernel<T, R, DV>), dim3(LV_GRID), dim3(LV_THREADS), 0, s,
                           a);
    } else {
        hipLaunchKernelGGL((level_seg_kernel<T, R, DV, true>), sg, dim3(LV_THREADS), 0, s, a);
        hipLaunchKernelGGL((level_keys_kernel<T, R, DV>), dim3(LV_GRID), dim3(LV_THREADS), 0, s,
                           a);
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
