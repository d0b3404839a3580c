// dism_scan.hip -- label scans: the length-1 part of every valid pair, in O(N) per (b,h).
//
// Every valid pair (key j <= query i, equal labels) is first treated as a length-1 match
// with weight p1 = exp2(LUT[1] - m_i); pairs with L >= 2 (bigram pairs, dism_pairs.hip)
// carry the corrections.  The length-1 part factorises through per-label running matrices
//   forward / dSQ:  M_i[r][d] = sum over valid keys j of sk_j[r] * v_j[d]
//   dSK / dV:       N_j[r][d] = sum over valid queries i of (p1_i sq_i[r]) * dO_i[d]
// so one pass over each label group replaces the pairwise sweep.  The combined label order
// (dism_sort.hip) lists a group's keys and queries already merged in position order.
//
// Mapping (MI355X): one 64-lane wave per (b,h) row and top-digit bucket (one label when
// labels are below 256).  The group streams through windows of WIN entries:
//   * per-entry work that does not depend on the running matrix (positions, key counts by
//     ballot prefix, exp2/log2/reciprocals of the row statistics, the tau formula) is done
//     lane-parallel, one entry per lane, once per window;
//   * value rows (v or dO) are copied HBM -> LDS with global_load_lds_dwordx4 into a double
//     buffer, readout rows are converted to fp32 in LDS, and window k+1's loads are in
//     flight while window k is consumed;
//   * the running matrix lives in registers in one of two lane layouts: "column" (lane = d,
//     all R rows per lane: products over r are lane-local) or "row-group" (lane = r*G + g,
//     G = 64/R, VPL = DV/G consecutive columns per lane: products over d reduce over the G
//     lanes of a row with in-row DPP adds).
//
// fp32 sequences (the CPU model repeats them):
//   M, N: fma chains over the group's entries in merge order (N in DESCENDING position);
//   y[d] = chain_r fma(sq[r], M[r][d]);  dv0[d] = chain_r fma(sk[r], N[r][d]);
//   zq[r] = tree_g(chain_t fma(dO[gV+t], M[r][gV+t])) with V = VPL, tree_g the pairwise tree
//   over g = 0..G-1;  dsk0[r] = lane tree (lane_transpose_sum) of the per-lane terms
//   fma(N[r][l+64], v[l+64], N[r][l]*v[l]) (DV = 128) or N[r][l]*v[l] (0 beyond DV).
#include "dism_path.h"

DISM_TU_LAYOUT(scan)

namespace dism {

// ---------------------------------------------------------------------------------------
// Window bookkeeping over entries [lo, hi) of the combined order, ascending or descending.
template <int WIN, bool DESC>
struct Walk {
    const int32_t* ord;
    int lo, hi, nwin, k;
    int entC, entN, entP;  // lane-staged entries of windows k, k+1, k+2
    __device__ __forceinline__ int idx(int kk, int e) const {
        return DESC ? hi - 1 - kk * WIN - e : lo + kk * WIN + e;
    }
    __device__ __forceinline__ int count(int kk) const {
        const int r = (hi - lo) - kk * WIN;
        return r < WIN ? r : WIN;
    }
    __device__ __forceinline__ int load(int kk) const {
        const int lane = lane_id(), c = count(kk);
        const int e = lane < c ? lane : c - 1;
        return ord[idx(kk, e < WIN ? e : WIN - 1)];
    }
    __device__ __forceinline__ void begin(int lo_, int hi_) {
        // wave-uniform bounds in scalar registers: the entry loops then branch on scalars
        // instead of running as divergent loops with exec-mask bookkeeping
        lo = __builtin_amdgcn_readfirstlane(lo_);
        hi = __builtin_amdgcn_readfirstlane(hi_);
        nwin = (hi - lo + WIN - 1) / WIN;
        k = 0;
        entC = load(0);
        entN = nwin > 1 ? load(1) : 0;
        entP = nwin > 2 ? load(2) : 0;
    }
    // rotate after window k is done; returns false at the end
    __device__ __forceinline__ bool rotate() {
        ++k;
        if (k >= nwin) return false;
        entC = entN;
        entN = entP;
        if (k + 2 < nwin) entP = load(k + 2);
        return true;
    }
};

struct Item {
    int bh, b, h, bucket;
    long so, row0;
};

// work item = (b,h) row and top-digit bucket; grid = B*H*256 rounded up to a multiple of 8
__device__ __forceinline__ bool scan_item(const PathArgs& a, Item& it) {
    const int item = xcd_work_item();
    it.bh = item >> 8;
    if (it.bh >= a.B * a.H) return false;
    // dense hard rows are computed whole by the tile kernels (dism_dense.hip) or the level
    // kernels (dism_levels.hip)
    const int dmode = a.o.dflag[it.bh];
    if (pairless_mode(dmode) && a.hard[it.bh]) return false;
    it.bucket = item & 255;
    it.b = it.bh / a.H;
    it.h = it.bh - it.b * a.H;
    it.so = (long)it.bh * a.n;
    it.row0 = (long)it.b * a.n * a.H + it.h;
    return true;
}

// Runs of equal labels inside the bucket's range [c0, c1) of the combined order.
template <typename F>
__device__ __forceinline__ void for_runs(const int32_t* clab, int c0, int c1, F&& run) {
    int rs = __builtin_amdgcn_readfirstlane(c0);
    c1 = __builtin_amdgcn_readfirstlane(c1);
    while (rs < c1) {
        const uint32_t lbl = (uint32_t)__builtin_amdgcn_readfirstlane(clab[rs]);
        const int re = __builtin_amdgcn_readfirstlane(
            (uint32_t)clab[c1 - 1] == lbl ? c1 : upper_label(clab, rs + 1, c1, lbl));
        run(rs, re);
        rs = re;
    }
}

// ---------------------------------------------------------------------------------------
// forward.  Rows without bigram pairs are finished here:
//   out[d] = fma(p1, y[d], 0) * (1/den),  den = exp2(-m) + cnt*p1,  m = max(0, LUT[1]) if
//   cnt > 0 else 0;  rows with pairs get y and cnt in their record for the pair kernel.
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void scan_forward_kernel(PathArgs a) {
    using G_ = Geo<T, DV, 3072>;
    constexpr int WIN = G_::WIN, RB = G_::RB, NI = G_::NI;
    constexpr int COLS = (DV + 63) / 64;
    constexpr int W = words_of(sizeof(T), R);
    __shared__ __attribute__((aligned(16))) unsigned char s_v_all[WAVES][2][G_::BYTES];
    auto& s_v = s_v_all[wave_id()];
    __shared__ __attribute__((aligned(16))) float s_r_all[WAVES][WIN][R];
    auto& s_r = s_r_all[wave_id()];
    __shared__ int s_slot_all[WAVES][WIN];
    auto& s_slot = s_slot_all[wave_id()];
    // predecessor-label histogram of the current label group's keys, one 32-bit count per
    // predecessor byte (one-byte labels), for the pair counts computed here (fwd_phase 1)
    __shared__ uint32_t s_h_all[WAVES][256];
    uint32_t* s_h = s_h_all[wave_id()];
    Item it;
    if (!scan_item(a, it)) return;
    // fwd_phase 1: rows whose labels differ in one byte, pair counts from the histogram;
    // 2: the other rows, pair counts from the plan (pnb); 0: every row from pnb
    const int onebyte = a.fwd_phase ? a.o.onebyte[it.bh] : 0;
    if ((a.fwd_phase == 1 && !onebyte) || (a.fwd_phase == 2 && onebyte)) return;
    const bool hist_nb = a.fwd_phase == 1;
    const int lshift = hist_nb ? a.o.shift[it.bh] : 0;
    const int lane = lane_id();
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    const int32_t* corder = a.o.corder + 2 * it.so;
    const int32_t* clab = a.o.clab + 2 * it.so;
    const int32_t* ctab = a.o.ctab + (long)it.bh * 257;
    const int c0 = ctab[it.bucket], c1 = ctab[it.bucket + 1];
    if (c0 >= c1) return;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const unsigned char* vb = reinterpret_cast<const unsigned char*>(a.v);
    auto store_out = [&](long orow, int c, float val) {
        const int d = lane + 64 * c;
        if (d >= DV) return;
        if (a.out_dtype == DTYPE_F32)
            reinterpret_cast<float*>(a.out)[orow * DV + d] = val;
        else
            reinterpret_cast<uint16_t*>(a.out)[orow * DV + d] = (uint16_t)f32_to_bf16_bits(val);
    };

    if (!a.hard[it.bh]) {
        for (int t = c0; t < c1; ++t) {
            const int ent = corder[t];
            if (!(ent & 1)) continue;
            const int i = ent >> 1;
            const long orow = it.row0 + (long)i * a.H;
#pragma unroll
            for (int c = 0; c < COLS; ++c) store_out(orow, c, 0.0f);
            if (lane == 0) {
                a.lse2[it.so + i] = 0.0f;
                if (a.lmax) a.lmax[it.so + i] = 0;
                if (a.jarg) a.jarg[it.so + i] = -1;
            }
        }
        return;
    }
    const float lut1 = a.lut[(long)it.h * a.lut_stride + 1];

    for_runs(clab, c0, c1, [&](int rs, int re) {
        Walk<WIN, false> wk;
        wk.ord = corder;
        wk.begin(rs, re);
        // per-lane data of window k+1 (issued one window ahead) and of window k
        uint32_t wN[W];
        int nbN = 0;  // pair count of the query row, or the predecessor's label byte (-1: none)
        auto issue = [&](int kk, int ent) {  // readout words, pair count, key rows -> s_v
            const int p = ent >> 1;
            const bool isq = ent & 1;
            load_words<W>((isq ? sq : sk) + (it.row0 + (long)p * a.H) * R, wN);
            if (hist_nb)
                nbN = p >= 1 ? (int)(((uint32_t)(isq ? a.iq : a.ik)[it.so + p - 1] >> lshift) &
                                     255u)
                             : -1;
            else
                nbN = isq ? a.pnb[it.so + p] : 0;
            const bool ok = lane < wk.count(kk);
            const unsigned long long km = __ballot(ok && !isq);
            const int nk = __popcll(km);
            if (ok && !isq) s_slot[__popcll(km & below)] = p;
            if (nk > 0)
                dma_rows<RB, NI>((lds_u8*)s_v[kk & 1], nk, [&](int s) {
                    return vb + (it.row0 + (long)s_slot[s] * a.H) * RB;
                });
        };
        issue(0, wk.entC);
        uint32_t wC[W];
        int nbC;
#pragma unroll
        for (int c = 0; c < W; ++c) wC[c] = wN[c];
        nbC = nbN;
        if (wk.nwin > 1) issue(1, wk.entN);
        wait_vm0();

        float M[R][COLS];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < COLS; ++c) M[r][c] = 0.0f;
        int carry_cnt = 0, carry_last = -1;
        if (hist_nb) {
            for (int x = lane; x < 256; x += 64) s_h[x] = 0u;
            asm volatile("" ::: "memory");
        }
        do {
            const int kk = wk.k, wn = __builtin_amdgcn_readfirstlane(wk.count(kk));
            // ---- lane-parallel: entry kind, key counts, row statistics, fp32 readout rows
            const int ent = wk.entC, p = ent >> 1;
            const bool ok = lane < wn, isq = ok && (ent & 1);
            const unsigned long long km = __ballot(ok && !isq), qm = __ballot(isq);
            const int cnt = carry_cnt + __popcll(km & below);
            const unsigned long long kb = km & below;
            const int hl = kb ? 63 - __clzll(kb) : 0;
            const int lastk = __shfl(p, hl);
            const int last = kb ? lastk : carry_last;
            {
                float rr[R];
#pragma unroll
                for (int r = 0; r < R; ++r) rr[r] = word_elem<T>(wC, r);
                if (ok) {
#pragma unroll
                    for (int r = 0; r < R; ++r) s_r[lane][r] = rr[r];
                }
            }
            int nb = nbC;
            if (hist_nb) {
                // bigram partners of a query: the group's keys before it (j >= 1) whose
                // predecessor label equals the query's -- earlier windows from the histogram,
                // this window's from the lanes before it; then this window's keys join the
                // histogram
                const int pl = nbC;
                int c = 0;
                if (isq && pl >= 0) c = (int)s_h[pl];
                // only keys before the window's last query can count
                const unsigned long long qv = __ballot(isq && pl >= 0);
                unsigned long long kv = __ballot(ok && !isq && pl >= 0);
                kv = qv ? kv & (~0ull >> __clzll(qv)) : 0ull;  // lanes up to the last query
                while (kv) {
                    const int l = __ffsll((long long)kv) - 1;
                    kv &= kv - 1;
                    const int pll = readlane_i(pl, l);  // uniform: read by every lane
                    if (isq && l < lane && pl == pll) ++c;
                }
                nb = isq ? c : 0;
                asm volatile("" ::: "memory");
                if (ok && !isq && pl >= 0) atomicAdd(&s_h[pl], 1u);
                asm volatile("" ::: "memory");
            }
            const float m = (cnt > 0 && lut1 > 0.0f) ? lut1 : 0.0f;
            const float p1 = exp2_fp32(lut1 - m);
            const float den = exp2_fp32(-m) + (float)cnt * p1;
            const float rden = 1.0f / den;
            if (isq) {
                if (nb == 0) {
                    a.lse2[it.so + p] = m + log2_fp32(den);
                    if (a.lmax) a.lmax[it.so + p] = cnt > 0 ? 1 : 0;
                    if (a.jarg) a.jarg[it.so + p] = cnt > 0 ? last : -1;
                } else {
                    a.prow[(it.so + p) * a.prow_stride + PREC_CNT] = __int_as_float(cnt);
                }
            }
            const int nkeys = __popcll(km);
            const unsigned long long hk = km;
            carry_cnt += nkeys;
            if (hk) carry_last = __shfl(p, 63 - __clzll(hk));
            // ---- the merge (window k+1's loads are in flight): keys update M, queries emit
            const unsigned char* vbuf = s_v[kk & 1];
            int slot = 0;
            for (int e = 0; e < wn; ++e) {
                float rr[R];
                lds_row_f32<R>(&s_r[e][0], rr);
                const bool qe = (qm >> e) & 1;
                if (qe) {
                    float y[COLS];
#pragma unroll
                    for (int c = 0; c < COLS; ++c) {
                        y[c] = 0.0f;
#pragma unroll
                        for (int r = 0; r < R; ++r) y[c] = __builtin_fmaf(rr[r], M[r][c], y[c]);
                    }
                    const int i = readlane_i(p, e);
                    if (readlane_i(nb, e) == 0) {
                        const float p1e = readlane_f(p1, e), rde = readlane_f(rden, e);
                        const long orow = it.row0 + (long)i * a.H;
#pragma unroll
                        for (int c = 0; c < COLS; ++c)
                            store_out(orow, c, __builtin_fmaf(p1e, y[c], 0.0f) * rde);
                    } else {
                        float* rec = a.prow + (it.so + i) * a.prow_stride + PREC_Y;
#pragma unroll
                        for (int c = 0; c < COLS; ++c)
                            if (lane + 64 * c < DV) rec[lane + 64 * c] = y[c];
                    }
                }
                // two one-sided branches kept apart (an if/else made the compiler copy the
                // running matrix on every entry): read M, then update M in place
                asm volatile("" ::: "memory");
                if (!qe) {
                    const unsigned char* row = vbuf + slot * RB;
                    ++slot;
                    float vv[COLS];
#pragma unroll
                    for (int c = 0; c < COLS; ++c)
                        vv[c] = lane + 64 * c < DV ? lds_elem<T>(row, lane + 64 * c) : 0.0f;
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int c = 0; c < COLS; ++c) M[r][c] = __builtin_fmaf(rr[r], vv[c], M[r][c]);
                }
            }
            if (!wk.rotate()) break;
            wait_vm0();
#pragma unroll
            for (int c = 0; c < W; ++c) wC[c] = wN[c];
            nbC = nbN;
            if (wk.k + 1 < wk.nwin) issue(wk.k + 1, wk.entN);
        } while (true);
    });
}

// ---------------------------------------------------------------------------------------
// backward, query rows: dSQ and the per-row tau term (row corrections from the pair kernel).
// Row-group layout: lane = r*G + g holds M[r][g*VPL .. g*VPL+VPL).
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void scan_rows_kernel(PathArgs a) {
    using G_ = Geo<T, DV, 3072>;
    constexpr int WIN = G_::WIN, RB = G_::RB, NI = G_::NI;
    constexpr int W = words_of(sizeof(T), R);
    constexpr int G = 64 / R, VPL = DV / G;
    __shared__ __attribute__((aligned(16))) unsigned char s_v_all[WAVES][2][G_::BYTES];
    auto& s_v = s_v_all[wave_id()];
    __shared__ __attribute__((aligned(16))) float s_r_all[WAVES][WIN][R];
    auto& s_r = s_r_all[wave_id()];
    __shared__ __attribute__((aligned(16))) float s_z_all[WAVES][WIN][R];
    auto& s_z = s_z_all[wave_id()];
    Item it;
    if (!scan_item(a, it)) return;
    const int lane = lane_id(), rl = lane / G, gl = lane % G;
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    const int32_t* corder = a.o.corder + 2 * it.so;
    const int32_t* clab = a.o.clab + 2 * it.so;
    const int32_t* ctab = a.o.ctab + (long)it.bh * 257;
    const int c0 = ctab[it.bucket], c1 = ctab[it.bucket + 1];
    if (c0 >= c1) return;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const unsigned char* vb = reinterpret_cast<const unsigned char*>(a.v);
    const unsigned char* db = reinterpret_cast<const unsigned char*>(a.dout);

    if (!a.hard[it.bh]) {
        for (int t = c0 + lane; t < c1; t += 64) {
            const int ent = corder[t];
            if (!(ent & 1)) continue;
            const int i = ent >> 1;
            float* g = a.dsq + (it.row0 + (long)i * a.H) * R;
#pragma unroll
            for (int r = 0; r < R; ++r) g[r] = 0.0f;
            a.rowtau[it.so + i] = 0.0f;
        }
        return;
    }
    const float* lut = a.lut + (long)it.h * a.lut_stride;
    const float* glut = a.dlut + (long)it.h * a.lut_stride;
    const float lut1 = lut[1], glut1 = glut[1];
    constexpr int NX = 3 + R + 4;  // lse2, G[i+1], pair count, cdq[R], cu, cvv, cw, cz

    for_runs(clab, c0, c1, [&](int rs, int re) {
        Walk<WIN, false> wk;
        wk.ord = corder;
        wk.begin(rs, re);
        uint32_t wN[W], xN[NX];
        auto issue = [&](int kk, int ent) {
            const int p = ent >> 1;
            const bool isq = ent & 1;
            load_words<W>((isq ? sq : sk) + (it.row0 + (long)p * a.H) * R, wN);
            // row statistics only for query entries, corrections only for rows with pairs
            xN[0] = isq ? __float_as_uint(a.lse2[it.so + p]) : 0u;
            xN[1] = isq ? __float_as_uint(glut[p - doc_start(a, p) + 1]) : 0u;
            xN[2] = isq ? (uint32_t)a.pnb[it.so + p] : 0u;
            const float* rec = a.prow + (it.so + p) * a.prow_stride;
            const bool has = isq && xN[2] > 0;
#pragma unroll
            for (int x = 0; x < R + 4; ++x) xN[3 + x] = has ? __float_as_uint(rec[x]) : 0u;
            const int n_ok = wk.count(kk);
            dma_rows<RB, NI>((lds_u8*)s_v[kk & 1], n_ok, [&](int s) {
                const int es = __shfl(ent, s);
                return ((es & 1) ? db : vb) + (it.row0 + (long)(es >> 1) * a.H) * RB;
            });
        };
        issue(0, wk.entC);
        uint32_t wC[W], xC[NX];
#pragma unroll
        for (int c = 0; c < W; ++c) wC[c] = wN[c];
#pragma unroll
        for (int c = 0; c < NX; ++c) xC[c] = xN[c];
        if (wk.nwin > 1) issue(1, wk.entN);
        wait_vm0();

        float M[VPL];
#pragma unroll
        for (int t = 0; t < VPL; ++t) M[t] = 0.0f;
        int carry_cnt = 0;
        do {
            const int kk = wk.k, wn = __builtin_amdgcn_readfirstlane(wk.count(kk));
            const int ent = wk.entC, p = ent >> 1;
            const bool ok = lane < wn, isq = ok && (ent & 1);
            const unsigned long long km = __ballot(ok && !isq), qm = __ballot(isq);
            const int cnt = carry_cnt + __popcll(km & below);
            carry_cnt += __popcll(km);
            const int nb = (int)xC[2];
            const bool has = isq && nb > 0;
            {
                float rr[R];
#pragma unroll
                for (int r = 0; r < R; ++r) rr[r] = word_elem<T>(wC, r);
                if (ok) {
#pragma unroll
                    for (int r = 0; r < R; ++r) s_r[lane][r] = rr[r];
                }
            }
            const float l2 = __uint_as_float(xC[0]);
            const float cc = __uint_as_float(xC[1]);
            const float P1 = exp2_fp32(lut1 - l2);
            const float q1 = P1 * (glut1 - cc);
            const float cu = has ? __uint_as_float(xC[3 + R]) : 0.0f;
            const float cvv = has ? __uint_as_float(xC[4 + R]) : 0.0f;
            const float cw = has ? __uint_as_float(xC[5 + R]) : 0.0f;
            const float cz = has ? __uint_as_float(xC[6 + R]) : 0.0f;
            const unsigned char* vbuf = s_v[kk & 1];
            for (int e = 0; e < wn; ++e) {
                const unsigned char* row = vbuf + e * RB + gl * VPL * (int)sizeof(T);
                float vals[VPL];
                lds_vals<T, VPL>(row, vals);
                const bool qe = (qm >> e) & 1;
                if (qe) {
                    // zq[r] of this query to LDS; dSQ and the tau terms are finished
                    // lane-parallel (one query per lane) after the window
                    float part = 0.0f;
#pragma unroll
                    for (int t = 0; t < VPL; ++t) part = __builtin_fmaf(vals[t], M[t], part);
                    const float zq = group_sum<G>(part);
                    if (gl == 0) s_z[e][rl] = zq;
                }
                asm volatile("" ::: "memory");  // one-sided branches (see scan_forward_kernel)
                if (!qe) {
                    const float s = s_r[e][rl];
#pragma unroll
                    for (int t = 0; t < VPL; ++t) M[t] = __builtin_fmaf(s, vals[t], M[t]);
                }
            }
            asm volatile("" ::: "memory");
            if (isq) {
                float zq[R], rr[R], g[R];
                lds_row_f32<R>(&s_z[lane][0], zq);
#pragma unroll
                for (int r = 0; r < R; ++r) rr[r] = word_elem<T>(wC, r);
                float se0v = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    se0v = __builtin_fmaf(rr[r], zq[r], se0v);
                    g[r] = __builtin_fmaf(P1, zq[r], has ? __uint_as_float(xC[3 + r]) : 0.0f);
                }
                store_row_f32<R>(a.dsq + (it.row0 + (long)p * a.H) * R, g);
                const float fc = (float)cnt;
                const float uu = __builtin_fmaf(P1, se0v, cu);
                const float vv = __builtin_fmaf(fc, q1, cvv);
                const float ww = __builtin_fmaf(q1, se0v, cw);
                const float z = __builtin_fmaf(fc, P1, cz);
                const float f = exp2_fp32(-l2);
                const float mass = z + f;
                const float mean = __builtin_fmaf(-f, cc, vv) / mass;
                a.rowtau[it.so + p] = __builtin_fmaf(-uu, mean, ww) / mass;
            }
            if (!wk.rotate()) break;
            wait_vm0();
#pragma unroll
            for (int c = 0; c < W; ++c) wC[c] = wN[c];
#pragma unroll
            for (int c = 0; c < NX; ++c) xC[c] = xN[c];
            if (wk.k + 1 < wk.nwin) issue(wk.k + 1, wk.entN);
        } while (true);
    });
}

// ---------------------------------------------------------------------------------------
// backward, keys: the length-1 parts dSK0, dV0 (pair corrections are added afterwards by the
// key pair kernel).  Merge in DESCENDING position order: a query at the key's own position
// comes before the key.  N is kept in the column layout (lane = d); dSK0 reduces over lanes.
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void scan_keys_kernel(PathArgs a) {
    using G_ = Geo<T, DV, WBYTES / 2>;  // half windows: 70 VGPRs, LDS allows 7 waves/SIMD
    constexpr int WIN = G_::WIN, RB = G_::RB, NI = G_::NI;
    constexpr int COLS = (DV + 63) / 64;
    constexpr int W = words_of(sizeof(T), R);
    constexpr int G = 64 / R;
    __shared__ __attribute__((aligned(16))) unsigned char s_v_all[WAVES][2][G_::BYTES];
    auto& s_v = s_v_all[wave_id()];
    __shared__ __attribute__((aligned(16))) float s_r_all[WAVES][WIN][R];
    auto& s_r = s_r_all[wave_id()];
    Item it;
    if (!scan_item(a, it)) return;
    const int lane = lane_id(), rl = lane / G, gl = lane % G;
    const int32_t* corder = a.o.corder + 2 * it.so;
    const int32_t* clab = a.o.clab + 2 * it.so;
    const int32_t* ctab = a.o.ctab + (long)it.bh * 257;
    const int c0 = ctab[it.bucket], c1 = ctab[it.bucket + 1];
    if (c0 >= c1) return;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const unsigned char* vb = reinterpret_cast<const unsigned char*>(a.v);
    const unsigned char* db = reinterpret_cast<const unsigned char*>(a.dout);

    if (!a.hard[it.bh]) {
        for (int t = c0; t < c1; ++t) {
            const int ent = corder[t];
            if (ent & 1) continue;
            const long krow = it.row0 + (long)(ent >> 1) * a.H;
#pragma unroll
            for (int c = 0; c < COLS; ++c) {
                const int d = lane + 64 * c;
                if (d < DV) a.dv[krow * DV + d] = 0.0f;
            }
            if (lane < R) a.dsk[krow * R + lane] = 0.0f;
        }
        return;
    }
    const float lut1 = a.lut[(long)it.h * a.lut_stride + 1];

    for_runs(clab, c0, c1, [&](int rs, int re) {
        Walk<WIN, true> wk;
        wk.ord = corder;
        wk.begin(rs, re);
        uint32_t wN[W];
        float lN;
        auto issue = [&](int kk, int ent) {
            const int p = ent >> 1;
            const bool isq = ent & 1;
            load_words<W>((isq ? sq : sk) + (it.row0 + (long)p * a.H) * R, wN);
            lN = isq ? a.lse2[it.so + p] : 0.0f;
            dma_rows<RB, NI>((lds_u8*)s_v[kk & 1], wk.count(kk), [&](int s) {
                const int es = __shfl(ent, s);
                return ((es & 1) ? db : vb) + (it.row0 + (long)(es >> 1) * a.H) * RB;
            });
        };
        issue(0, wk.entC);
        uint32_t wC[W];
        float lC;
#pragma unroll
        for (int c = 0; c < W; ++c) wC[c] = wN[c];
        lC = lN;
        if (wk.nwin > 1) issue(1, wk.entN);
        wait_vm0();

        float Nd[R][COLS];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int c = 0; c < COLS; ++c) Nd[r][c] = 0.0f;
        do {
            const int kk = wk.k, wn = __builtin_amdgcn_readfirstlane(wk.count(kk));
            const int ent = wk.entC, p = ent >> 1;
            const bool ok = lane < wn, isq = ok && (ent & 1);
            const unsigned long long qm = __ballot(isq);
            {
                // keys: sk; queries: a[r] = exp2(LUT[1] - lse2) * sq[r]
                const float P1 = exp2_fp32(lut1 - lC);
                if (ok) {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float x = word_elem<T>(wC, r);
                        s_r[lane][r] = isq ? P1 * x : x;
                    }
                }
            }
            const unsigned char* vbuf = s_v[kk & 1];
            for (int e = 0; e < wn; ++e) {
                const unsigned char* row = vbuf + e * RB;
                float rr[R];
                lds_row_f32<R>(&s_r[e][0], rr);
                const bool qe = (qm >> e) & 1;
                // the entry's value row in the column layout (v for a key, dO for a query)
                float vd[COLS];
#pragma unroll
                for (int c = 0; c < COLS; ++c)
                    vd[c] = lane + 64 * c < DV ? lds_elem<T>(row, lane + 64 * c) : 0.0f;
                if (!qe) {
                    // key: dV0 = sk . N (lane-local); dSK0 = N . v over d, from per-lane
                    // partial products summed across the wave by lane_transpose_sum
                    const int j = readlane_i(p, e);
                    const long krow = it.row0 + (long)j * a.H;
                    float part[R];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        part[r] = Nd[r][0] * vd[0];
#pragma unroll
                        for (int c = 1; c < COLS; ++c) part[r] = __builtin_fmaf(Nd[r][c], vd[c], part[r]);
                    }
#pragma unroll
                    for (int c = 0; c < COLS; ++c) {
                        float y = 0.0f;
#pragma unroll
                        for (int r = 0; r < R; ++r) y = __builtin_fmaf(rr[r], Nd[r][c], y);
                        if (lane + 64 * c < DV) a.dv[krow * DV + lane + 64 * c] = y;
                    }
                    const float dk = lane_transpose_sum<R>(part);
                    if (gl == 0) a.dsk[krow * R + rl] = dk;
                }
                // keeps the two one-sided branches apart (an if/else here made the compiler
                // copy the running matrix on every entry)
                asm volatile("" ::: "memory");
                if (qe) {
                    // query: N += a (x) dO (column layout, lane = d)
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int c = 0; c < COLS; ++c) Nd[r][c] = __builtin_fmaf(rr[r], vd[c], Nd[r][c]);
                }
            }
            if (!wk.rotate()) break;
            wait_vm0();
#pragma unroll
            for (int c = 0; c < W; ++c) wC[c] = wN[c];
            lC = lN;
            if (wk.k + 1 < wk.nwin) issue(wk.k + 1, wk.entN);
        } while (true);
    });
}

// ---------------------------------------------------------------------------------------
#define DISM_SCAN_LAUNCHER(NAME, KERNEL)                                                      \
    template <typename T, int R, int DV>                                                      \
    static hipError_t NAME##_go(const PathArgs& a, hipStream_t s) {                           \
        const long items = 256L * a.B * a.H;                                                  \
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

DISM_SCAN_LAUNCHER(scan_forward, scan_forward_kernel)
DISM_SCAN_LAUNCHER(scan_rows, scan_rows_kernel)
DISM_SCAN_LAUNCHER(scan_keys, scan_keys_kernel)

}  // namespace dism
