// dism_prefix.h -- prefix rows (mode 4): dense hard rows in which every label has one
// predecessor label (all-identical labels, a period of distinct labels).
//
// In such a row a valid pair (i, j <= i, iq[i] == ik[j]) with j >= 1 has iq[i-1] == ik[j-1],
// so its match runs back to the key's row start: L_ij = j + 1.  The weight of a pair,
// exp2(LUT[j+1] - m_i), is then a function of the key alone (up to the query's maximum m_i),
// and a query's sum over its valid keys is a prefix sum over its label group.  The reference
// computes these rows with the same O(N^2) pairwise loop as every other row
// (dism_v3/src/hard_forward.cu:28-118, hard_backward.cu:26-154); here they cost O(N R DV)
// (the prefix matrices) plus O(N x 32) pairwise work inside 64-entry segments.
//
// The list is the combined label order (corder: entries e = 2p + s sorted by (label, p, s)),
// cut into segments of PREFIX_SEG = 64 entries; one wave holds a segment, lane = entry slot.
//   prefix_tot_kernel    per segment: the weighted key sum T_s of its last group piece
//                        relative to the piece's largest weight M_s (forward and query side),
//                        or the query sum U_s of its first piece (key side);
//   prefix_chain_kernel  per row, sequential over segments: the state before each segment
//                        (running maximum mu, P = sum of T_s rescaled to mu), restarting at
//                        group starts; the key side runs descending with a running minimum
//                        of lse2;
//   prefix_forward_kernel / prefix_rows_kernel / prefix_keys_kernel  per segment: every query
//                        (key) starts from its segment's state when its group began earlier
//                        (continues later) and adds the pairs inside the segment one by one.
// Everything is a fixed fp32 sequence, restated by the oracle's prefix_forward_row /
// prefix_backward_row (oracle/dism_cpu_model.c), which spell out each step.  Lanes = value
// columns (DV <= 128: CPL = 1 or 2 per lane) for the matrices; the reductions over d use the
// column layout's transposing butterfly (lane_transpose_sum).
//
// A row is a prefix row when it is dense (dense_classify_kernel), has no query resets or
// documents, and every label bucket (the classification's 12-bit label hash) holds one label
// and, over positions >= 1 on either side, one predecessor label (dense_classify_kernel,
// dism_dense.hip).
#pragma once
#include "dism_path.h"

namespace dism {

constexpr int PX_THREADS = 128;
constexpr int PX_WAVES = PX_THREADS / 64;
constexpr unsigned PX_GRID = 1024;   // persistent workgroups of the segment kernels
constexpr int PX_EPT = 2;            // chain elements per thread
constexpr int PX_CHAIN_THREADS = 256;
constexpr int PX_MAX_SEGS = 2 * DENSE_MAX_N / PREFIX_SEG;
constexpr int PX_HAS = 1 << 20, PX_RESET = 1 << 21;

__device__ __forceinline__ int pxrl(int x, int t) { return __builtin_amdgcn_readlane(x, t); }
__device__ __forceinline__ float pxrlf(float x, int t) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), t));
}
__device__ __forceinline__ void px_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// xor-butterfly sum over the wave (every lane gets the same bits)
__device__ __forceinline__ float px_wave_tree(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = x + __shfl_xor(x, o);
    return x;
}

// ---------------------------------------------------------------------------------------
// One segment held by a wave: lane = entry slot.
struct PxSeg {
    int bh, b, h, n, nseg, s, x0, cnt;
    int e, lab, p;
    bool isk, isq, hasprev, hasnext;
    int prevlab, nextlab;
    long row;        // the lane's vector row (position p)
    long sbase;      // the segment's slot in the per-segment buffers (bh * nseg + s)
};

// positions a prefix row holds: a prefill's rows are padded after their first cls_n real
// tokens, and their list is the combined order without the padding (prefix_compact_kernel)
__device__ __forceinline__ int px_cn(const PathArgs& a) {
    return a.cls_n > 0 && a.cls_n < a.n ? a.cls_n : a.n;
}

__device__ __forceinline__ PxSeg px_seg(const PathArgs& a, int bh, int s) {
    PxSeg g;
    const int lane = lane_id();
    const int cn = px_cn(a);
    g.bh = bh;
    g.n = a.n;
    g.b = bh / a.H;
    g.h = bh - g.b * a.H;
    g.nseg = px_segs(a.n);  // the per-segment buffers' row stride
    g.s = s;
    const int n2 = 2 * cn;
    g.x0 = s * PREFIX_SEG;
    g.cnt = n2 - g.x0 < PREFIX_SEG ? n2 - g.x0 : PREFIX_SEG;
    const bool padded = cn < a.n;
    const int32_t* E = (padded ? a.o.pxE : a.o.corder) + (long)bh * 2 * a.n;
    const int32_t* LB = (padded ? a.o.pxL : a.o.clab) + (long)bh * 2 * a.n;
    const bool in = lane < g.cnt;
    g.e = in ? E[g.x0 + lane] : 0;
    g.lab = in ? LB[g.x0 + lane] : 0;
    g.p = g.e >> 1;
    g.isk = in && !(g.e & 1);
    g.isq = in && (g.e & 1);
    g.hasprev = s > 0;
    g.prevlab = g.hasprev ? LB[g.x0 - 1] : 0;
    g.hasnext = g.x0 + PREFIX_SEG < n2;
    g.nextlab = g.hasnext ? LB[g.x0 + PREFIX_SEG] : 0;
    g.row = ((long)g.b * a.n + g.p) * a.H + g.h;
    g.sbase = (long)bh * g.nseg + s;
    return g;
}

// copy NV elements of T from global row src to LDS row dst (lane-private rows)
template <typename T, int NV>
__device__ __forceinline__ void px_stage(unsigned char* dst, const T* src) {
    constexpr int BYTES = NV * (int)sizeof(T);
    if constexpr (BYTES % 16 == 0) {
#pragma unroll
        for (int c = 0; c < BYTES / 16; ++c)
            reinterpret_cast<uint4*>(dst)[c] = reinterpret_cast<const uint4*>(src)[c];
    } else if constexpr (BYTES % 8 == 0) {
#pragma unroll
        for (int c = 0; c < BYTES / 8; ++c)
            reinterpret_cast<uint2*>(dst)[c] = reinterpret_cast<const uint2*>(src)[c];
    } else if constexpr (BYTES % 4 == 0) {
#pragma unroll
        for (int c = 0; c < BYTES / 4; ++c)
            reinterpret_cast<uint32_t*>(dst)[c] = reinterpret_cast<const uint32_t*>(src)[c];
    } else {
#pragma unroll
        for (int c = 0; c < NV; ++c) reinterpret_cast<T*>(dst)[c] = src[c];
    }
}

template <typename T>
__device__ __forceinline__ float px_elem(const unsigned char* row, int d) {
    return lds_elem<T>(row, d);
}

// ---------------------------------------------------------------------------------------
// Segment totals.  KIND 0: forward (T, S, M, last key), 1: query side of the backward (also
// TB and SG), 2: key side (U over the first piece's queries, descending, and lambda).
template <typename T, int R, int DV, int KIND>
__global__ __launch_bounds__(PX_THREADS) void prefix_tot_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, ESZ = (int)sizeof(T);
    constexpr int RB = R * ESZ, VB = DV * ESZ;
    __shared__ __align__(16) unsigned char s_r[PX_WAVES][64 * RB];
    __shared__ __align__(16) unsigned char s_v[PX_WAVES][64 * VB];
    const int w = wave_id(), lane = lane_id();
    const int BH = a.B * a.H, nseg = px_segs(px_cn(a));
    const int rows = a.o.dcount[3];
    const long items = (long)rows * nseg;
    const long RD = (long)R * DV;
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long it = (long)blockIdx.x * PX_WAVES + w; it < items; it += (long)gridDim.x * PX_WAVES) {
        const int ri = (int)(it / nseg), s = (int)(it - (long)ri * nseg);
        const int bh = a.o.dlist[3 * BH + ri];
        if (!a.hard[bh]) continue;
        const PxSeg g = px_seg(a, bh, s);
        if constexpr (KIND < 2) {
            // last piece: the entries of the last entry's group (labels are contiguous)
            const int lastlab = pxrl(g.lab, g.cnt - 1);
            const bool inp = lane < g.cnt && g.lab == lastlab;
            const unsigned long long km = __ballot(inp && g.isk);
            const bool reset = !g.hasprev || g.prevlab != lastlab;
            const float* lut = a.lut + (long)g.h * a.lut_stride;
            const float ell = (inp && g.isk) ? lut[g.p + 1] : -INFINITY;
            float M = ell;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
            const float wt = exp2_fp32(ell - M);
            // backward: G - G0 with G0 the G of the piece's last key (the segment's centre)
            float gg = 0.0f;
            if constexpr (KIND == 1) {
                const float* dl = a.dlut + (long)g.h * a.lut_stride;
                const float g0 = km ? dl[pxrl(g.p, 63 - __builtin_clzll(km)) + 1] : 0.0f;
                gg = (inp && g.isk) ? dl[g.p + 1] - g0 : 0.0f;
            }
            if (inp && g.isk) {
                px_stage<T, R>(&s_r[w][lane * RB], sk + g.row * R);
                px_stage<T, DV>(&s_v[w][lane * VB], v + g.row * DV);
            }
            px_wave_sync();
            float acc[R][CPL], accb[KIND == 1 ? R : 1][CPL];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    acc[r][c] = 0.0f;
                    if constexpr (KIND == 1) accb[r][c] = 0.0f;
                }
            float S = 0.0f, SG = 0.0f;
            int K = -1;
            unsigned long long m = km;
            while (m) {
                const int t = __builtin_ctzll(m);
                m &= m - 1;
                const float wv = pxrlf(wt, t);
                float skr[R];
                lds_vals<T, R>(&s_r[w][t * RB], skr);
                float vc[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int col = lane + 64 * c;
                    vc[c] = col < DV ? px_elem<T>(&s_v[w][t * VB], col) : 0.0f;
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float ar = wv * skr[r];
#pragma unroll
                    for (int c = 0; c < CPL; ++c) acc[r][c] = __builtin_fmaf(ar, vc[c], acc[r][c]);
                }
                if constexpr (KIND == 1) {
                    const float gv = pxrlf(gg, t);
                    const float wg = wv * gv;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float br = wg * skr[r];
#pragma unroll
                        for (int c = 0; c < CPL; ++c)
                            accb[r][c] = __builtin_fmaf(br, vc[c], accb[r][c]);
                    }
                    SG = __builtin_fmaf(wv, gv, SG);
                }
                S = S + wv;
                K = pxrl(g.p, t);
            }
            float* T0 = a.o.pxT + g.sbase * RD;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int col = lane + 64 * c;
                    if (col < DV) T0[(long)r * DV + col] = acc[r][c];
                }
            if constexpr (KIND == 1) {
                float* B0 = a.o.pxB + g.sbase * RD;
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const int col = lane + 64 * c;
                        if (col < DV) B0[(long)r * DV + col] = accb[r][c];
                    }
            }
            if (lane == 0) {
                const int fl = (K + 1) | (km ? PX_HAS : 0) | (reset ? PX_RESET : 0);
                a.o.pxS[g.sbase] = make_float4(km ? M : 0.0f, S, SG, __int_as_float(fl));
            }
            px_wave_sync();
        } else {
            // first piece: the entries of the first entry's group
            const int firstlab = pxrl(g.lab, 0);
            const bool inp = lane < g.cnt && g.lab == firstlab;
            const unsigned long long qm = __ballot(inp && g.isq);
            const bool reset = !g.hasnext || g.nextlab != firstlab;
            const float l2 = (inp && g.isq) ? a.lse2[(long)bh * a.n + g.p] : INFINITY;
            float lam = l2;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) lam = fminf(lam, __shfl_xor(lam, o));
            const float wq = exp2_fp32(lam - l2);
            if (inp && g.isq) {
                px_stage<T, R>(&s_r[w][lane * RB], sq + g.row * R);
                px_stage<T, DV>(&s_v[w][lane * VB], dout + g.row * DV);
            }
            px_wave_sync();
            float acc[R][CPL];
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) acc[r][c] = 0.0f;
            unsigned long long m = qm;
            while (m) {
                const int t = 63 - __builtin_clzll(m);
                m &= ~(1ull << t);
                const float wv = pxrlf(wq, t);
                float sqr[R];
                lds_vals<T, R>(&s_r[w][t * RB], sqr);
                float dc[CPL];
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int col = lane + 64 * c;
                    dc[c] = col < DV ? px_elem<T>(&s_v[w][t * VB], col) : 0.0f;
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float ar = wv * sqr[r];
#pragma unroll
                    for (int c = 0; c < CPL; ++c) acc[r][c] = __builtin_fmaf(ar, dc[c], acc[r][c]);
                }
            }
            float* U0 = a.o.pxU + g.sbase * RD;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int col = lane + 64 * c;
                    if (col < DV) U0[(long)r * DV + col] = acc[r][c];
                }
            if (lane == 0) {
                const int fl = (qm ? 1 : 0) | (reset ? 2 : 0);
                a.o.pxK[g.sbase] = make_float2(qm ? lam : 0.0f, __int_as_float(fl));
            }
            px_wave_sync();
        }
    }
}

// ---------------------------------------------------------------------------------------
// Chains.  Block (row, chunk of PX_CHAIN_THREADS * PX_EPT elements).  Thread 0 runs the
// scalar chain into LDS (the per-segment factors g, h and an opcode: bit 0 restart, bit 1
// update / bit 2 set), then every thread walks its elements through the segments in order,
// writing the state before each segment over that segment's total.
template <int KIND>
__global__ __launch_bounds__(PX_CHAIN_THREADS) void prefix_chain_kernel(PathArgs a, int RD) {
    __shared__ float2 s_gh[PX_MAX_SEGS];
    __shared__ float s_dg[KIND == 1 ? PX_MAX_SEGS : 1];
    __shared__ uint8_t s_op[PX_MAX_SEGS];
    // the segments' records (and, KIND 1, the centre G0 of each), loaded in parallel so that
    // the sequential scalar chain below reads LDS only
    __shared__ float4 s_in[PX_MAX_SEGS];
    __shared__ float s_g0[KIND == 1 ? PX_MAX_SEGS : 1];
    __shared__ float2 s_m[PX_MAX_SEGS];
    const int bh = blockIdx.x, tid = threadIdx.x;
    if (a.o.dflag[bh] != 4 || !a.hard[bh]) return;
    const int nseg = px_segs(px_cn(a));
    const long sb = (long)bh * px_segs(a.n);
    for (int s = tid; s < nseg; s += PX_CHAIN_THREADS) {
        if constexpr (KIND < 2) {
            const float4 t = a.o.pxS[sb + s];
            s_in[s] = t;
            if constexpr (KIND == 1) {
                const int fl = __float_as_int(t.w);
                s_g0[s] = (fl & PX_HAS)
                              ? a.dlut[(long)(bh % a.H) * a.lut_stride + (fl & 0xFFFFF)]
                              : 0.0f;
            }
        } else {
            const float2 t = a.o.pxK[sb + s];
            s_in[s] = make_float4(t.x, t.y, 0.0f, 0.0f);
        }
    }
    __syncthreads();
    // (1) thread 0: the running maximum (minimum) alone, the base after a restart and the
    // value after each segment; (2) all threads: the factors g, h; (3) thread 0: the scalar
    // sums and the records of the state before (after) each segment
    if (tid == 0) {
        if constexpr (KIND < 2) {
            float mu = 0.0f;
            for (int s = 0; s < nseg; ++s) {
                const float4 t = s_in[s];
                const int fl = __float_as_int(t.w);
                int op = 0;
                if (fl & PX_RESET) {
                    mu = 0.0f;
                    op |= 1;
                }
                const float mb = mu;
                if (fl & PX_HAS) {
                    mu = t.x > mu ? t.x : mu;
                    op |= 2;
                }
                s_m[s] = make_float2(mb, mu);
                s_op[s] = (uint8_t)op;
            }
        } else {
            float nu = 0.0f;
            int has = 0;
            const bool wr = blockIdx.y == 0;
            for (int s = nseg - 1; s >= 0; --s) {
                const float4 t = s_in[s];
                const int fl = __float_as_int(t.y);
                if (wr) a.o.pxKR[sb + s] = make_float2(nu, __int_as_float(has));
                int op = 0;
                if (fl & 2) {
                    has = 0;
                    nu = 0.0f;
                    op |= 1;
                }
                const float nb = nu;
                if (fl & 1) {
                    if (!has) {
                        nu = t.x;
                        has = 1;
                        op |= 4;
                    } else {
                        nu = t.x < nu ? t.x : nu;
                        op |= 2;
                    }
                }
                s_m[s] = make_float2(nb, nu);
                s_op[s] = (uint8_t)op;
            }
        }
    }
    __syncthreads();
    for (int s = tid; s < nseg; s += PX_CHAIN_THREADS) {
        const int op = s_op[s];
        const float2 m = s_m[s];
        float g = 1.0f, h = 1.0f;
        if (op & 2) {
            if constexpr (KIND < 2) {
                g = exp2_fp32(m.x - m.y);
                h = exp2_fp32(s_in[s].x - m.y);
            } else {
                g = exp2_fp32(m.y - m.x);
                h = exp2_fp32(m.y - s_in[s].x);
            }
        }
        s_gh[s] = make_float2(g, h);
    }
    __syncthreads();
    if constexpr (KIND < 2) {
        if (tid == 0) {
            // KIND 0 keeps the last key in .w, KIND 1 the centre gam of the G-weighted sums
            float PS = 0.0f, PSG = 0.0f, gam = 0.0f, mu = 0.0f;
            int lk = -1;
            const bool wr = blockIdx.y == 0;
            for (int s = 0; s < nseg; ++s) {
                const float4 t = s_in[s];
                const int fl = __float_as_int(t.w);
                if (wr)
                    a.o.pxR[sb + s] =
                        make_float4(mu, PS, PSG, KIND == 1 ? gam : __int_as_float(lk));
                if (fl & PX_RESET) {
                    PS = 0.0f; PSG = 0.0f; gam = 0.0f; lk = -1;
                }
                float dG = 0.0f;
                if (fl & PX_HAS) {
                    const float2 gh = s_gh[s];
                    lk = (fl & 0xFFFFF) - 1;
                    if constexpr (KIND == 1) {
                        const float g0 = s_g0[s];
                        dG = gam - g0;
                        PSG = __builtin_fmaf(gh.y, t.z, __builtin_fmaf(dG, PS, PSG) * gh.x);
                        gam = g0;
                    }
                    PS = __builtin_fmaf(gh.y, t.y, PS * gh.x);
                }
                mu = s_m[s].y;
                if constexpr (KIND == 1) s_dg[s] = dG;
            }
        }
        __syncthreads();
    }
    float* A = KIND == 2 ? a.o.pxU : a.o.pxT;
    float* Bm = KIND == 1 ? a.o.pxB : nullptr;
    const long e0 = (long)blockIdx.y * PX_CHAIN_THREADS * PX_EPT + tid;
    float st[PX_EPT], sbv[PX_EPT];
    bool ok[PX_EPT];
#pragma unroll
    for (int x = 0; x < PX_EPT; ++x) {
        st[x] = 0.0f;
        sbv[x] = 0.0f;
        ok[x] = e0 + (long)x * PX_CHAIN_THREADS < RD;
    }
    constexpr int PF = 8;  // segments whose totals are loaded ahead
    for (int i0 = 0; i0 < nseg; i0 += PF) {
        float tv[PF][PX_EPT], tb[PF][PX_EPT];
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int i = i0 + u;
            const int s = KIND == 2 ? nseg - 1 - i : i;
#pragma unroll
            for (int x = 0; x < PX_EPT; ++x) {
                const long el = e0 + (long)x * PX_CHAIN_THREADS;
                const bool live = i < nseg && ok[x];
                tv[u][x] = live ? A[(sb + s) * RD + el] : 0.0f;
                if constexpr (KIND == 1) tb[u][x] = live ? Bm[(sb + s) * RD + el] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int i = i0 + u;
            if (i >= nseg) break;
            const int s = KIND == 2 ? nseg - 1 - i : i;
            const int op = s_op[s];
            const float2 gh = s_gh[s];
#pragma unroll
            for (int x = 0; x < PX_EPT; ++x) {
                if (!ok[x]) continue;
                const long el = e0 + (long)x * PX_CHAIN_THREADS;
                A[(sb + s) * RD + el] = st[x];
                if constexpr (KIND == 1) Bm[(sb + s) * RD + el] = sbv[x];
                if (op & 1) {
                    st[x] = 0.0f;
                    sbv[x] = 0.0f;
                }
                if (op & 2) {
                    if constexpr (KIND == 1)
                        sbv[x] = __builtin_fmaf(gh.y, tb[u][x],
                                                __builtin_fmaf(s_dg[s], st[x], sbv[x]) * gh.x);
                    st[x] = __builtin_fmaf(gh.y, tv[u][x], st[x] * gh.x);
                } else if (op & 4) {
                    st[x] = tv[u][x];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// Segmented inclusive maximum of x over the lanes of each label run (lane >= gstart).
__device__ __forceinline__ float px_run_max(float x, int gstart) {
    const int lane = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(x, o);
        if (lane - o >= gstart) x = fmaxf(x, y);
    }
    return x;
}
// first lane of the lane's label run
__device__ __forceinline__ int px_gstart(const PxSeg& g) {
    const int lane = lane_id();
    const int up = __shfl_up(g.lab, 1);
    const bool head = lane == 0 || up != g.lab;
    const unsigned long long hm = __ballot(head);
    const unsigned long long below = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
    return 63 - __builtin_clzll(hm & below);
}

// Forward, one wave per segment.  LDS: the key slots' value rows, the query slots' sq rows.
template <typename T, int R, int DV>
__global__ __launch_bounds__(PX_THREADS) void prefix_forward_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, ESZ = (int)sizeof(T);
    constexpr int RB = R * ESZ, VB = DV * ESZ;
    __shared__ __align__(16) unsigned char s_q[PX_WAVES][64 * RB];
    __shared__ __align__(16) unsigned char s_v[PX_WAVES][64 * VB];
    const int w = wave_id(), lane = lane_id();
    const int BH = a.B * a.H, nseg = px_segs(px_cn(a));
    const int rows = a.o.dcount[3];
    const long items = (long)rows * nseg;
    const long RD = (long)R * DV;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    for (long it = (long)blockIdx.x * PX_WAVES + w; it < items; it += (long)gridDim.x * PX_WAVES) {
        const int ri = (int)(it / nseg), s = (int)(it - (long)ri * nseg);
        const int bh = a.o.dlist[3 * BH + ri];
        if (!a.hard[bh]) continue;
        const PxSeg g = px_seg(a, bh, s);
        const unsigned long long kmask = __ballot(g.isk), qmask = __ballot(g.isq);
        if (!qmask) continue;
        const float* lut = a.lut + (long)g.h * a.lut_stride;
        const float ell = g.isk ? lut[g.p + 1] : -INFINITY;
        float skr[R];
        if (g.isk) {
            load_row<T, R>(sk + g.row * R, skr);
            px_stage<T, DV>(&s_v[w][lane * VB], v + g.row * DV);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) skr[r] = 0.0f;
        }
        if (g.isq) px_stage<T, R>(&s_q[w][lane * RB], sq + g.row * R);
        const int gst = px_gstart(g);
        const float pm = px_run_max(ell, gst);
        const bool anyuse = __ballot(g.isq && g.hasprev && g.lab == g.prevlab) != 0ull;
        float P[R][CPL];
        float4 pre = make_float4(0.0f, 0.0f, 0.0f, __int_as_float(-1));
        if (anyuse) {
            const float* P0 = a.o.pxT + g.sbase * RD;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int col = lane + 64 * c;
                    P[r][c] = col < DV ? P0[(long)r * DV + col] : 0.0f;
                }
            pre = a.o.pxR[g.sbase];
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) P[r][c] = 0.0f;
        }
        px_wave_sync();
        unsigned long long qm = qmask;
        while (qm) {
            const int xq = __builtin_ctzll(qm);
            qm &= qm - 1;
            const int lq = pxrl(g.lab, xq), pq = pxrl(g.p, xq);
            const bool use = g.hasprev && lq == g.prevlab;
            const unsigned long long eq = __ballot(g.lab == lq);
            const unsigned long long km = kmask & eq & ((1ull << xq) - 1ull);
            const float mub = use ? pre.x : 0.0f, psb = use ? pre.y : 0.0f;
            float m = mub;
            if (km) {
                const float pmx = pxrlf(pm, xq);
                m = pmx > m ? pmx : m;
            }
            const float f = exp2_fp32(mub - m);
            float den = __builtin_fmaf(psb, f, exp2_fp32(-m));
            float sqv[R];
            lds_vals<T, R>(&s_q[w][xq * RB], sqv);
            float y[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                float acc = 0.0f;
                if (use) {
#pragma unroll
                    for (int r = 0; r < R; ++r) acc = __builtin_fmaf(sqv[r], P[r][c], acc);
                }
                y[c] = use ? acc * f : 0.0f;
            }
            int jb = use ? __float_as_int(pre.w) : -1;
            if (km) {
                const float pr = exp2_fp32(ell - m);
                float sv = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) sv = __builtin_fmaf(sqv[r], skr[r], sv);
                const float ps = pr * sv;
                unsigned long long mm = km;
                int last = 0;
                while (mm) {
                    const int t = __builtin_ctzll(mm);
                    mm &= mm - 1;
                    den = den + pxrlf(pr, t);
                    const float pst = pxrlf(ps, t);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const int col = lane + 64 * c;
                        const float vv = col < DV ? px_elem<T>(&s_v[w][t * VB], col) : 0.0f;
                        y[c] = __builtin_fmaf(pst, vv, y[c]);
                    }
                    last = t;
                }
                jb = pxrl(g.p, last);
            }
            const long orow = (((long)g.b * a.n + pq) * a.H + g.h) * DV;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                if (col < DV) {
                    const float o = y[c] / den;
                    if (a.out_dtype == DTYPE_F32)
                        reinterpret_cast<float*>(a.out)[orow + col] = o;
                    else
                        reinterpret_cast<uint16_t*>(a.out)[orow + col] = (uint16_t)f32_to_bf16_bits(o);
                }
            }
            if (lane == 0) {
                const long qi = (long)bh * a.n + pq;
                a.lse2[qi] = m + log2_fp32(den);
                if (a.lmax) a.lmax[qi] = jb >= 0 ? jb + 1 : 0;
                if (a.jarg) a.jarg[qi] = jb;
            }
        }
        px_wave_sync();
    }
}

// Backward, query side: dSQ and the row's tau term.  LDS: the query slots' sq and dO rows,
// the key slots' value rows.
template <typename T, int R, int DV>
__global__ __launch_bounds__(PX_THREADS) void prefix_rows_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, ESZ = (int)sizeof(T);
    constexpr int RB = R * ESZ, VB = DV * ESZ;
    constexpr int G = 64 / R;
    __shared__ __align__(16) unsigned char s_q[PX_WAVES][64 * RB];
    __shared__ __align__(16) unsigned char s_d[PX_WAVES][64 * VB];
    __shared__ __align__(16) unsigned char s_v[PX_WAVES][64 * VB];
    const int w = wave_id(), lane = lane_id();
    const int BH = a.B * a.H, nseg = px_segs(px_cn(a));
    const int rows = a.o.dcount[3];
    const long items = (long)rows * nseg;
    const long RD = (long)R * DV;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long it = (long)blockIdx.x * PX_WAVES + w; it < items; it += (long)gridDim.x * PX_WAVES) {
        const int ri = (int)(it / nseg), s = (int)(it - (long)ri * nseg);
        const int bh = a.o.dlist[3 * BH + ri];
        if (!a.hard[bh]) continue;
        const PxSeg g = px_seg(a, bh, s);
        const unsigned long long kmask = __ballot(g.isk), qmask = __ballot(g.isq);
        if (!qmask) continue;
        const float* lut = a.lut + (long)g.h * a.lut_stride;
        const float* dl = a.dlut + (long)g.h * a.lut_stride;
        const float ell = g.isk ? lut[g.p + 1] : 0.0f;
        const float gk = g.isk ? dl[g.p + 1] : 0.0f;
        float skr[R];
        if (g.isk) {
            load_row<T, R>(sk + g.row * R, skr);
            px_stage<T, DV>(&s_v[w][lane * VB], v + g.row * DV);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) skr[r] = 0.0f;
        }
        if (g.isq) {
            px_stage<T, R>(&s_q[w][lane * RB], sq + g.row * R);
            px_stage<T, DV>(&s_d[w][lane * VB], dout + g.row * DV);
        }
        const bool anyuse = __ballot(g.isq && g.hasprev && g.lab == g.prevlab) != 0ull;
        float P[R][CPL], PB[R][CPL];
        float4 pre = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (anyuse) {
            const float* P0 = a.o.pxT + g.sbase * RD;
            const float* B0 = a.o.pxB + g.sbase * RD;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int col = lane + 64 * c;
                    P[r][c] = col < DV ? P0[(long)r * DV + col] : 0.0f;
                    PB[r][c] = col < DV ? B0[(long)r * DV + col] : 0.0f;
                }
            pre = a.o.pxR[g.sbase];
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    P[r][c] = 0.0f;
                    PB[r][c] = 0.0f;
                }
        }
        px_wave_sync();
        unsigned long long qm = qmask;
        while (qm) {
            const int xq = __builtin_ctzll(qm);
            qm &= qm - 1;
            const int lq = pxrl(g.lab, xq), pq = pxrl(g.p, xq);
            const bool use = g.hasprev && lq == g.prevlab;
            const unsigned long long eq = __ballot(g.lab == lq);
            const unsigned long long km = kmask & eq & ((1ull << xq) - 1ull);
            const long qi = (long)bh * a.n + pq;
            const float l2 = a.lse2[qi], cc = dl[pq + 1];
            const float kap = exp2_fp32((use ? pre.x : 0.0f) - l2);
            float sqv[R];
            lds_vals<T, R>(&s_q[w][xq * RB], sqv);
            float dcol[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                dcol[c] = col < DV ? px_elem<T>(&s_d[w][xq * VB], col) : 0.0f;
            }
            // prefix part: zP[r] and zB[r] by the column layout's transposing butterfly
            float zP = 0.0f, zB = 0.0f;
            if (use) {
                float x1[R], x2[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    x1[r] = dcol[0] * P[r][0];
                    x2[r] = dcol[0] * PB[r][0];
                    if constexpr (CPL == 2) {
                        x1[r] = __builtin_fmaf(dcol[1], P[r][1], x1[r]);
                        x2[r] = __builtin_fmaf(dcol[1], PB[r][1], x2[r]);
                    }
                }
                zP = lane_transpose_sum<R>(x1);
                zB = lane_transpose_sum<R>(x2);
            }
            // lane r*G holds zP[r], zB[r]
            const bool rl = (lane % G) == 0;
            const int rr = lane / G;
            const float sqr = lds_elem<T>(&s_q[w][xq * RB], rr);
            const float u0 = px_wave_tree(rl ? sqr * zP : 0.0f) * kap;
            const float W0 = px_wave_tree(rl ? sqr * zB : 0.0f) * kap;
            const float z0 = (use ? pre.y : 0.0f) * kap, zg0 = (use ? pre.z : 0.0f) * kap;
            const float cg = cc - (use ? pre.w : 0.0f);
            const float vv0 = __builtin_fmaf(-cg, z0, zg0), w0 = __builtin_fmaf(-cg, u0, W0);
            // own keys, lane = slot
            const bool own = (km >> lane) & 1ull;
            float tA = 0.0f, tB = 0.0f, tC = 0.0f, tD = 0.0f;
            float xk[R];
#pragma unroll
            for (int r = 0; r < R; ++r) xk[r] = 0.0f;
            if (km) {
                const float p = exp2_fp32(ell - l2);
                float sv = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) sv = __builtin_fmaf(sqv[r], skr[r], sv);
                float ev = 0.0f;
                {
                    constexpr int CH = DV < 16 ? DV : 16;
                    const unsigned char* vrow = &s_v[w][lane * VB];
                    const unsigned char* drow = &s_d[w][xq * VB];
#pragma unroll
                    for (int d0 = 0; d0 < DV; d0 += CH) {
                        float vr[CH], dr[CH];
                        lds_vals<T, CH>(vrow + d0 * ESZ, vr);
                        lds_vals<T, CH>(drow + d0 * ESZ, dr);
#pragma unroll
                        for (int d = 0; d < CH; ++d) ev = __builtin_fmaf(dr[d], vr[d], ev);
                    }
                }
                const float ps = p * sv, pe = p * ev, pse = ps * ev, gg = gk - cc;
                if (own) {
                    tA = pse;
                    tB = p * gg;
                    tC = pse * gg;
                    tD = p;
#pragma unroll
                    for (int r = 0; r < R; ++r) xk[r] = pe * skr[r];
                }
            }
            const float u = u0 + px_wave_tree(tA), vv = vv0 + px_wave_tree(tB);
            const float ww = w0 + px_wave_tree(tC), z = z0 + px_wave_tree(tD);
            const float dqp = km ? lane_transpose_sum<R>(xk) : 0.0f;
            const float dq = zP * kap + dqp;
            if (rl && rr < R) a.dsq[(((long)g.b * a.n + pq) * a.H + g.h) * R + rr] = dq;
            if (lane == 0) {
                const float f = exp2_fp32(-l2), mass = z + f;
                const float mean = __builtin_fmaf(-f, cc, vv) / mass;
                a.rowtau[qi] = __builtin_fmaf(-u, mean, ww) / mass;
            }
        }
        px_wave_sync();
    }
}

// Backward, key side: dSK and dV.  LDS: the query slots' dO rows, the key slots' sk and value
// rows.
template <typename T, int R, int DV>
__global__ __launch_bounds__(PX_THREADS) void prefix_keys_kernel(PathArgs a) {
    constexpr int CPL = (DV + 63) / 64, ESZ = (int)sizeof(T);
    constexpr int RB = R * ESZ, VB = DV * ESZ;
    constexpr int G = 64 / R;
    __shared__ __align__(16) unsigned char s_k[PX_WAVES][64 * RB];
    __shared__ __align__(16) unsigned char s_d[PX_WAVES][64 * VB];
    __shared__ __align__(16) unsigned char s_v[PX_WAVES][64 * VB];
    const int w = wave_id(), lane = lane_id();
    const int BH = a.B * a.H, nseg = px_segs(px_cn(a));
    const int rows = a.o.dcount[3];
    const long items = (long)rows * nseg;
    const long RD = (long)R * DV;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long it = (long)blockIdx.x * PX_WAVES + w; it < items; it += (long)gridDim.x * PX_WAVES) {
        const int ri = (int)(it / nseg), s = (int)(it - (long)ri * nseg);
        const int bh = a.o.dlist[3 * BH + ri];
        if (!a.hard[bh]) continue;
        const PxSeg g = px_seg(a, bh, s);
        const unsigned long long kmask = __ballot(g.isk), qmask = __ballot(g.isq);
        if (!kmask) continue;
        const float* lut = a.lut + (long)g.h * a.lut_stride;
        const float l2 = g.isq ? a.lse2[(long)bh * a.n + g.p] : 0.0f;
        float sqr[R];
        if (g.isq) {
            load_row<T, R>(sq + g.row * R, sqr);
            px_stage<T, DV>(&s_d[w][lane * VB], dout + g.row * DV);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) sqr[r] = 0.0f;
        }
        if (g.isk) {
            px_stage<T, R>(&s_k[w][lane * RB], sk + g.row * R);
            px_stage<T, DV>(&s_v[w][lane * VB], v + g.row * DV);
        }
        const bool anyuse = __ballot(g.isk && g.hasnext && g.lab == g.nextlab) != 0ull;
        float Q[R][CPL];
        float2 suf = make_float2(0.0f, 0.0f);
        if (anyuse) {
            suf = a.o.pxKR[g.sbase];
            const float* Q0 = a.o.pxU + g.sbase * RD;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const int col = lane + 64 * c;
                    Q[r][c] = col < DV ? Q0[(long)r * DV + col] : 0.0f;
                }
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int c = 0; c < CPL; ++c) Q[r][c] = 0.0f;
        }
        const bool sufhas = __float_as_int(suf.y) != 0;
        px_wave_sync();
        unsigned long long kq = kmask;
        while (kq) {
            const int xk = __builtin_ctzll(kq);
            kq &= kq - 1;
            const int lk = pxrl(g.lab, xk), pk = pxrl(g.p, xk);
            const bool use = g.hasnext && lk == g.nextlab && sufhas;
            const unsigned long long eq = __ballot(g.lab == lk);
            const unsigned long long qm = qmask & eq & ~((2ull << xk) - 1ull);
            const float lj = lut[pk + 1];
            float skv[R];
            lds_vals<T, R>(&s_k[w][xk * RB], skv);
            float vcol[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                vcol[c] = col < DV ? px_elem<T>(&s_v[w][xk * VB], col) : 0.0f;
            }
            float dvv[CPL];
            float dk = 0.0f;
            if (use) {
                const float phi = exp2_fp32(lj - suf.x);
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    float acc = 0.0f;
#pragma unroll
                    for (int r = 0; r < R; ++r) acc = __builtin_fmaf(skv[r], Q[r][c], acc);
                    dvv[c] = acc * phi;
                }
                float x1[R];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    x1[r] = vcol[0] * Q[r][0];
                    if constexpr (CPL == 2) x1[r] = __builtin_fmaf(vcol[1], Q[r][1], x1[r]);
                }
                dk = lane_transpose_sum<R>(x1) * phi;
            } else {
#pragma unroll
                for (int c = 0; c < CPL; ++c) dvv[c] = 0.0f;
            }
            if (qm) {
                const bool own = (qm >> lane) & 1ull;
                const float p = exp2_fp32(lj - l2);
                float sv = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) sv = __builtin_fmaf(sqr[r], skv[r], sv);
                float ev = 0.0f;
                {
                    constexpr int CH = DV < 16 ? DV : 16;
                    const unsigned char* drow = &s_d[w][lane * VB];
                    const unsigned char* vrow = &s_v[w][xk * VB];
#pragma unroll
                    for (int d0 = 0; d0 < DV; d0 += CH) {
                        float vr[CH], dr[CH];
                        lds_vals<T, CH>(vrow + d0 * ESZ, vr);
                        lds_vals<T, CH>(drow + d0 * ESZ, dr);
#pragma unroll
                        for (int d = 0; d < CH; ++d) ev = __builtin_fmaf(dr[d], vr[d], ev);
                    }
                }
                const float ps = p * sv, pe = p * ev;
                float x2[R];
#pragma unroll
                for (int r = 0; r < R; ++r) x2[r] = own ? pe * sqr[r] : 0.0f;
                dk = dk + lane_transpose_sum<R>(x2);
                unsigned long long mm = qm;
                while (mm) {
                    const int t = __builtin_ctzll(mm);
                    mm &= mm - 1;
                    const float pst = pxrlf(ps, t);
#pragma unroll
                    for (int c = 0; c < CPL; ++c) {
                        const int col = lane + 64 * c;
                        const float dd = col < DV ? px_elem<T>(&s_d[w][t * VB], col) : 0.0f;
                        dvv[c] = __builtin_fmaf(pst, dd, dvv[c]);
                    }
                }
            }
            const long krow = ((long)g.b * a.n + pk) * a.H + g.h;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int col = lane + 64 * c;
                if (col < DV) a.dv[krow * DV + col] = dvv[c];
            }
            const int rr = lane / G;
            if ((lane % G) == 0 && rr < R) a.dsk[krow * R + rr] = dk;
        }
        px_wave_sync();
    }
}

// ---------------------------------------------------------------------------------------
// A padded prefill row's list: the combined order's entries of the first cls_n positions, in
// order (block-wide ballot scan per 1024-entry chunk).
template <int UNUSED>
__global__ __launch_bounds__(1024) void prefix_compact_kernel(PathArgs a) {
    __shared__ int s_w[16];
    const int bh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (a.o.dflag[bh] != 4) return;
    const int n2 = 2 * a.n, cn = px_cn(a);
    const int32_t* E = a.o.corder + (long)bh * n2;
    const int32_t* LB = a.o.clab + (long)bh * n2;
    int32_t* oE = a.o.pxE + (long)bh * n2;
    int32_t* oL = a.o.pxL + (long)bh * n2;
    int base = 0;
    for (int c0 = 0; c0 < n2; c0 += 1024) {
        const int x = c0 + tid;
        const int e = x < n2 ? E[x] : 0;
        const bool keep = x < n2 && (e >> 1) < cn;
        const unsigned long long m = __ballot(keep);
        if (lane == 0) s_w[w] = __popcll(m);
        __syncthreads();
        int off = base;
        for (int v = 0; v < w; ++v) off += s_w[v];
        if (keep) {
            const int at = off + __popcll(m & ((1ull << lane) - 1ull));
            oE[at] = e;
            oL[at] = LB[x];
        }
        int t = 0;
        for (int v = 0; v < 16; ++v) t += s_w[v];
        base += t;
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------
// launchers: WHICH 0 forward, 1 backward query side, 2 backward key side (one translation
// unit each: dism_prefix.hip, dism_prefix_rows.hip, dism_prefix_keys.hip)
template <int WHICH, typename T, int R, int DV>
static hipError_t prefix_go(const PathArgs& a, hipStream_t s) {
    const unsigned BH = (unsigned)(a.B * a.H);
    const int RD = R * DV;
    const dim3 cg(BH, (unsigned)((RD + PX_CHAIN_THREADS * PX_EPT - 1) / (PX_CHAIN_THREADS * PX_EPT)));
    if constexpr (WHICH == 0) {
        if (a.cls_n > 0 && a.cls_n < a.n)
            hipLaunchKernelGGL(prefix_compact_kernel<0>, dim3(BH), dim3(1024), 0, s, a);
    }
    hipLaunchKernelGGL((prefix_tot_kernel<T, R, DV, WHICH>), dim3(PX_GRID), dim3(PX_THREADS), 0, s, a);
    hipLaunchKernelGGL((prefix_chain_kernel<WHICH>), cg, dim3(PX_CHAIN_THREADS), 0, s, a, RD);
    if constexpr (WHICH == 0)
        hipLaunchKernelGGL((prefix_forward_kernel<T, R, DV>), dim3(PX_GRID), dim3(PX_THREADS), 0, s,
                           a);
    else if constexpr (WHICH == 1)
        hipLaunchKernelGGL((prefix_rows_kernel<T, R, DV>), dim3(PX_GRID), dim3(PX_THREADS), 0, s, a);
    else
        hipLaunchKernelGGL((prefix_keys_kernel<T, R, DV>), dim3(PX_GRID), dim3(PX_THREADS), 0, s, a);
    return hipGetLastError();
}

template <int WHICH, typename T, int R>
static hipError_t prefix_dv(const PathArgs& a, int DV, hipStream_t s) {
    switch (DV) {
        case 32: return prefix_go<WHICH, T, R, 32>(a, s);
        case 64: return prefix_go<WHICH, T, R, 64>(a, s);
        case 128: return prefix_go<WHICH, T, R, 128>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <int WHICH, typename T>
static hipError_t prefix_r(const PathArgs& a, int R, int DV, hipStream_t s) {
    switch (R) {
        case 2: return prefix_dv<WHICH, T, 2>(a, DV, s);
        case 4: return prefix_dv<WHICH, T, 4>(a, DV, s);
        case 8: return prefix_dv<WHICH, T, 8>(a, DV, s);
        case 16: return prefix_dv<WHICH, T, 16>(a, DV, s);
        case 32: return prefix_dv<WHICH, T, 32>(a, DV, s);
        default: return hipErrorInvalidValue;
    }
}

template <int WHICH>
static hipError_t prefix_launch(const PathArgs& a, int R, int DV, int dtype, hipStream_t s) {
    if (!a.o.pxT || a.dstart || a.wlo || a.n > DENSE_MAX_N) return hipSuccess;
    if (dtype == DTYPE_BF16) return prefix_r<WHICH, bf16_t>(a, R, DV, s);
    if (dtype == DTYPE_F32) return prefix_r<WHICH, float>(a, R, DV, s);
    return hipErrorInvalidValue;
}

}  // namespace dism
