// dism_dense.hip -- dense rows: hard rows whose labels collide often, computed with the
// direct (pairwise) definition over 64 x 32 query-key tiles.
//
// A row is dense when its bucketed label collisions M = sum over 4096 label buckets of
// #queries x #keys exceed N^2/64 (dense_classify_kernel; N <= DENSE_MAX_N).  Such rows have
// Theta(N^2) valid pairs: identical labels, tiny alphabets (d_qk = 2), long periodic runs.
// On them the label scans (dism_scan.hip) would run serially over one huge label group and
// the bigram walks (dism_pairs.hip) would cost O(pairs x L) = O(N^3).  Here every causal cell
// costs O(1) integer work for its match length and O(R + DV) floating point work, like the
// reference's quadratic path (dism_v3/src/hard_forward.cu, hard_backward.cu).
//
// Match lengths: the diagonal recurrence L[i,j] = (q[i] == k[j]) ? L[i-1,j-1] + 1 : 0
// (reset to 1 at a query reset / document start).  dense_bound_kernel sweeps each band of 64
// diagonals once (lane = diagonal, one query row per step) and stores the boundary rows
// L[64s - 1, j] (16-bit) of every 64-row query strip s.  A tile then rebuilds its lengths from
// its strip's boundary row: one thread per diagonal crossing the tile walks the strip's 64
// rows (dense_lengths).
//
// fp32 sequences (oracle/dism_cpu_model.c direct_forward_row / direct_backward_row):
//   forward, per query i, keys j ascending over valid pairs:
//     m = max(0, LUT[L]); den = exp2(-m); p = exp2(LUT[L] - m); den = den + p;
//     s = chain_r fma(sq[r], sk[r]); acc[d] = fma(p*s, v[d], acc[d]);
//     out = acc / den; lse2 = m + log2(den); longest match ties -> largest j.
//   backward, l2 = lse2_i, c = G[i - doc + 1]:  p = exp2(LUT[L] - l2);
//     s = chain_r fma(sq[r], sk[r]); e = chain_d fma(dO[d], v[d]); ps = p*s; pe = p*e;
//     pse = ps*e; g = G[L] - c;
//     per query (j ascending): dq[r] = fma(pe, sk[r], dq[r]); u = u + pse;
//       vv = fma(p, g, vv); w = fma(pse, g, w); z = z + p;
//       rowtau = fma(-u, mean, w) / mass, f = exp2(-l2), mass = z + f,
//       mean = fma(-f, c, vv) / mass;
//     per key (i ascending): dk[r] = fma(pe, sq[r], dk[r]); dv[d] = fma(ps, dO[d], dv[d]).
// A tile computes the per-pair scalars lane-parallel (phase A) into LDS, then folds them in
// order (phase B, lanes = accumulator elements).  Invalid cells contribute exact zeros
// (accumulators start at +0 and are never -0, so +0 terms are exact no-ops) unless a staged
// row holds a non-finite value; then phase B skips invalid cells explicitly.
#include "dism_path.h"

namespace dism {

constexpr int DENSE_THREADS = 256;
constexpr int DK = 32;              // keys per tile
constexpr unsigned DENSE_GRID = 512;   // persistent workgroups of the tile kernels

__device__ __forceinline__ uint32_t label_bucket(int32_t x) {
    return ((uint32_t)x * 0x9E3779B1u) >> 20;
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long x, int m) {
    const int lo = __shfl_xor((int)(uint32_t)x, m), hi = __shfl_xor((int)(uint32_t)(x >> 32), m);
    return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
}

// ---------------------------------------------------------------------------------------
// Classification: one workgroup per (b,h) row of n positions, counting the first cn of them
// (a prefill's rows are padded after the real tokens); bucket counts in LDS (runs of equal
// buckets in a thread's 16 consecutive labels are added with one atomic).
__global__ __launch_bounds__(256) void dense_classify_kernel(
    const int32_t* __restrict__ iq, const int32_t* __restrict__ ik, int n, int cn,
    int32_t* __restrict__ dflag, unsigned long long* __restrict__ dcost) {
    __shared__ uint32_t s_cnt[2][DENSE_BUCKETS];
    __shared__ unsigned long long s_red[4];
    const int tid = threadIdx.x;
    const long bh = blockIdx.x;
    for (int x = tid; x < 2 * DENSE_BUCKETS; x += 256) (&s_cnt[0][0])[x] = 0u;
    __syncthreads();
#pragma unroll
    for (int side = 0; side < 2; ++side) {
        const int32_t* lab = (side ? ik : iq) + bh * n;
        uint32_t* cnt = s_cnt[side];
        for (int base = tid * 16; base < cn; base += 256 * 16) {
            const int end = base + 16 < cn ? base + 16 : cn;
            uint32_t cur = label_bucket(lab[base]), c = 1;
            for (int x = base + 1; x < end; ++x) {
                const uint32_t bk = label_bucket(lab[x]);
                if (bk != cur) {
                    atomicAdd(&cnt[cur], c);
                    cur = bk;
                    c = 0;
                }
                ++c;
            }
            atomicAdd(&cnt[cur], c);
        }
    }
    __syncthreads();
    unsigned long long m = 0;
    for (int x = tid; x < DENSE_BUCKETS; x += 256)
        m += (unsigned long long)s_cnt[0][x] * s_cnt[1][x];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m += shfl_xor_u64(m, o);
    if ((tid & 63) == 0) s_red[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
        dcost[bh] = 0ull;  // the walk probe adds to it
        const unsigned long long t = s_red[0] + s_red[1] + s_red[2] + s_red[3];
        dflag[bh] =
            (n <= DENSE_MAX_N && t * 64ull > (unsigned long long)cn * (unsigned long long)cn)
                ? 1 : 0;
    }
}

// Row modes and lists (one workgroup, after the walk probe): mode 2 for the sparse rows
// whose walk-cost estimate exceeds N^2; the mode-1 rows ascending in dlist[0..), the rows of
// modes 1 and 2 ascending in dlist[BH..), their counts in dcount[0], dcount[1].
__global__ __launch_bounds__(1024) void dense_mode_kernel(int32_t* __restrict__ dflag,
                                                          const unsigned long long* __restrict__ dcost,
                                                          int BH, int n,
                                                          int32_t* __restrict__ dlist,
                                                          int32_t* __restrict__ dcount) {
    __shared__ int s_w[2][16];
    __shared__ int s_base[2];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const unsigned long long nn = (unsigned long long)n * (unsigned long long)n;
    if (tid < 2) s_base[tid] = 0;
    __syncthreads();
    for (int c0 = 0; c0 < BH; c0 += 1024) {
        const int x = c0 + tid;
        int mode = x < BH ? dflag[x] : 0;
        if (x < BH && mode == 0 && n <= DENSE_MAX_N && n > 64 && dcost[x] > nn) {
            mode = 2;
            dflag[x] = 2;
        }
        const unsigned long long m1 = __ballot(mode == 1), m2 = __ballot(mode != 0);
        if (lane == 0) {
            s_w[0][w] = __popcll(m1);
            s_w[1][w] = __popcll(m2);
        }
        __syncthreads();
        int b1 = s_base[0], b2 = s_base[1];
        for (int v = 0; v < w; ++v) {
            b1 += s_w[0][v];
            b2 += s_w[1][v];
        }
        const unsigned long long below = (1ull << lane) - 1ull;
        if (mode == 1) dlist[b1 + __popcll(m1 & below)] = x;
        if (mode != 0) dlist[BH + b2 + __popcll(m2 & below)] = x;
        __syncthreads();
        if (tid < 2) {
            int t = 0;
            for (int v = 0; v < 16; ++v) t += s_w[tid][v];
            s_base[tid] += t;
        }
        __syncthreads();
    }
    if (tid < 2) dcount[tid] = s_base[tid];
}

// query i starts its match afresh (query reset or document start)
__device__ __forceinline__ int dense_reset(const PathArgs& a, long so, int i) {
    if (!a.dstart && !a.wlo) return 0;
    return walk_lo(a, so, i) == i ? 1 : 0;
}

__device__ __forceinline__ const uint16_t* dense_strip(const PathArgs& a, int bh, int qs) {
    if (qs <= 0) return nullptr;
    return a.o.dbound + (long)bh * dense_row_entries(a.n) + dense_strip_offset(qs);
}

// ---------------------------------------------------------------------------------------
// Boundary rows: wave per (row of mode 1 or 2, band of 64 diagonals), persistent.  Lane l follows
// diagonal d = 64 band + l (cells (t, t - d)); labels are staged 64 steps at a time.
__global__ __launch_bounds__(256) void dense_bound_kernel(PathArgs a) {
    __shared__ int s_q[4][64], s_r[4][64], s_k[4][128];
    const int w = (int)(threadIdx.x >> 6), lane = (int)(threadIdx.x & 63);
    const int n = a.n, Q = (n + 63) >> 6;
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[1]);
    const long items = (long)cnt * Q;
    const int tend = 64 * (Q - 1) - 1;  // last boundary row
    const int32_t* rows = a.o.dlist + (long)a.B * a.H;
    for (long x = (long)blockIdx.x * 4 + w; x < items; x += (long)gridDim.x * 4) {
        const int band = (int)(x / cnt);
        const int bh = rows[x % cnt];
        const int d0 = 64 * band;
        if (d0 > tend) continue;  // (soft rows too: a prepare call has no row flags)
        const long so = (long)bh * n;
        const int32_t* q = a.iq + so;
        const int32_t* k = a.ik + so;
        uint16_t* bnd = a.o.dbound + (long)bh * dense_row_entries(n);
        const int delta = d0 + lane;
        int L = 0;
        for (int t0 = d0; t0 <= tend; t0 += 64) {
            {
                const int t = t0 + lane;
                s_q[w][lane] = t < n ? q[t] : 0;
                s_r[w][lane] = t < n ? dense_reset(a, so, t) : 0;
                int j = t0 - d0 - 63 + lane;
                s_k[w][lane] = (j >= 0 && j < n) ? k[j] : 0;
                j += 64;
                s_k[w][lane + 64] = (j >= 0 && j < n) ? k[j] : 0;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll 8
            for (int st = 0; st < 64; ++st) {
                const int j = t0 + st - delta;
                const bool eq = j >= 0 && s_q[w][st] == s_k[w][st - lane + 63];
                L = eq ? (s_r[w][st] ? 1 : L + 1) : 0;
            }
            const int j = t0 + 63 - delta;  // the boundary row of strip (t0 + 64) / 64
            if (j >= 0) bnd[dense_strip_offset((t0 + 64) >> 6) + j] = (uint16_t)L;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
}

// ---------------------------------------------------------------------------------------
// Tile lengths: the 64 x KT tile (rows i0 + il, keys j0 + jl) into sL[il * (KT + 1) + jl]
// (0 for non-causal cells and rows past n).  Thread t < 63 + KT walks the diagonal
// il - jl = t - (KT - 1) down the strip's 64 rows from the boundary row i0 - 1.
// sk holds the labels of keys j0 - 64 .. j0 + KT - 1 (sk[jl + 64]).
template <int KT>
__device__ __forceinline__ void dense_lengths(const int* sq, const int* sr, const int* sk,
                                              int* sL, int i0, int j0, int nq, int n,
                                              const uint16_t* bstrip, int tid) {
    if (tid >= 63 + KT) return;
    const int dl = tid - (KT - 1);
    const int jc = j0 - 1 - dl;
    int L = (bstrip && jc >= 0 && jc < i0) ? (int)bstrip[jc] : 0;
    for (int il = 0; il < 64; ++il) {
        const int jl = il - dl, j = j0 + jl;
        const bool in = jl < KT;
        const int kv = in ? sk[jl + 64] : 0;
        const bool eq = in && il < nq && j >= 0 && j < n && sq[il] == kv;
        L = eq ? (sr[il] ? 1 : L + 1) : 0;
        if (jl >= 0 && in) sL[il * (KT + 1) + jl] = (j <= i0 + il) ? L : 0;
    }
}

// Stage `rows` rows of width W (elements of T) as fp32 into dst[row][W]; source row x at
// src + (row0 + pos(x) * H) * W; rows with pos(x) outside [0, n) are zero.  Returns (via the
// workgroup) whether every staged value is finite.
template <typename T, int W, typename Pos>
__device__ __forceinline__ bool stage_rows(float* dst, const T* src, long row0, long H,
                                           int rows, int n, Pos pos, int tid) {
    constexpr int E = (int)(16 / sizeof(T)) < W ? (int)(16 / sizeof(T)) : W;
    constexpr int CH = W / E;  // chunks per row
    bool fin = true;
    for (int c = tid; c < rows * CH; c += DENSE_THREADS) {
        const int x = c / CH, col = (c - x * CH) * E;
        const int p = pos(x);
        float f[E];
        if (p >= 0 && p < n) {
            load_row<T, E>(src + (row0 + (long)p * H) * W + col, f);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) f[e] = 0.0f;
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            fin = fin && (__builtin_fabsf(f[e]) <= 3.402823466e38f);
            dst[x * W + col + e] = f[e];
        }
    }
    return __syncthreads_and(fin ? 1 : 0) != 0;
}

template <int N>
__device__ __forceinline__ void lds_vec(const float* p, float (&out)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int c = 0; c < N / 4; ++c) {
            const float4 x = reinterpret_cast<const float4*>(p)[c];
            out[4 * c] = x.x; out[4 * c + 1] = x.y; out[4 * c + 2] = x.z; out[4 * c + 3] = x.w;
        }
    } else if constexpr (N % 2 == 0) {
#pragma unroll
        for (int c = 0; c < N / 2; ++c) {
            const float2 x = reinterpret_cast<const float2*>(p)[c];
            out[2 * c] = x.x; out[2 * c + 1] = x.y;
        }
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) out[c] = p[c];
    }
}

__device__ __forceinline__ void lds4(const float* p, float (&o)[4]) {
    const float4 x = *reinterpret_cast<const float4*>(p);
    o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w;
}

// persistent item order: the longest strips first
struct DenseItem {
    int bh, strip;
};
__device__ __forceinline__ DenseItem dense_item(const PathArgs& a, long x, int cnt, int S,
                                                bool desc) {
    DenseItem it;
    const int s = (int)(x / cnt);
    it.strip = desc ? S - 1 - s : s;
    it.bh = a.o.dlist[x % cnt];
    return it;
}

template <typename T>
__device__ __forceinline__ void store_out(void* out, int out_dtype, long idx, const float* x,
                                          int cnt) {
    if (out_dtype == DTYPE_F32) {
        float* o = reinterpret_cast<float*>(out) + idx;
        for (int c = 0; c < cnt; ++c) o[c] = x[c];
    } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(out) + idx;
        for (int c = 0; c < cnt; ++c) o[c] = (uint16_t)f32_to_bf16_bits(x[c]);
    }
}

// ---------------------------------------------------------------------------------------
// forward: workgroup per (dense row, 64-query strip), key tiles of DK ascending; pass 1 the
// row shift m and the longest match, pass 2 the readout.
template <typename T, int R, int DV>
__global__ __launch_bounds__(DENSE_THREADS) void dense_forward_kernel(PathArgs a) {
    constexpr int KT = DK, KS = KT + 1, CPT = DV / 16, KG = KT / 4;
    __shared__ int s_qlab[64], s_rst[64], s_klab[KT + 64];
    __shared__ int s_L[64 * KS];
    __shared__ __attribute__((aligned(16))) float s_sk[KT * R];
    __shared__ __attribute__((aligned(16))) float s_v[KT * DV];
    __shared__ __attribute__((aligned(16))) float s_c[KT * 64];
    __shared__ __attribute__((aligned(16))) float s_p[KT * 64];
    __shared__ float s_m[64], s_den[64];
    __shared__ float s_pm[4][64];
    __shared__ unsigned long long s_key[4][64];
    const int tid = (int)threadIdx.x, l = tid & 63, g = tid >> 6;
    const int qq = tid & 15, cg = tid >> 4;
    const int n = a.n, Q = (n + 63) >> 6;
    const int cnt = __builtin_amdgcn_readfirstlane(*a.o.dcount);
    const long items = (long)cnt * Q;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    for (long x = blockIdx.x; x < items; x += gridDim.x) {
        const DenseItem it = dense_item(a, x, cnt, Q, true);
        const int bh = it.bh, qs = it.strip;
        if (!a.hard[bh]) continue;
        const int b = bh / a.H, h = bh - b * a.H;
        const long so = (long)bh * n, row0 = (long)b * n * a.H + h;
        const int i0 = qs * 64, nq = n - i0 < 64 ? n - i0 : 64;
        const uint16_t* bstrip = dense_strip(a, bh, qs);
        const float* lut = a.lut + (long)h * a.lut_stride;
        const int nkt = (i0 + nq + KT - 1) / KT;
        __syncthreads();
        if (tid < 64) {
            s_qlab[tid] = tid < nq ? a.iq[so + i0 + tid] : 0;
            s_rst[tid] = tid < nq ? dense_reset(a, so, i0 + tid) : 0;
        }
        float sqr[R];
        load_row<T, R>(sq + (row0 + (long)(l < nq ? i0 + l : i0) * a.H) * R, sqr);
        auto stage_keys = [&](int j0) {
            if (tid < KT + 64) {
                const int j = j0 - 64 + tid;
                s_klab[tid] = (j >= 0 && j < n) ? a.ik[so + j] : 0;
            }
        };
        // ---- pass 1: m = max(0, LUT[L]), longest match (ties -> largest key)
        float m = 0.0f;
        int best = 0, bj = -1;
        for (int kt = 0; kt < nkt; ++kt) {
            const int j0 = kt * KT;
            __syncthreads();
            stage_keys(j0);
            __syncthreads();
            dense_lengths<KT>(s_qlab, s_rst, s_klab, s_L, i0, j0, nq, n, bstrip, tid);
            __syncthreads();
#pragma unroll
            for (int u = 0; u < KG; ++u) {
                const int jl = g * KG + u;
                const int L = s_L[l * KS + jl];
                if (L > 0) {
                    const float lw = lut[L];
                    if (lw > m) m = lw;
                    if (L >= best) {
                        best = L;
                        bj = j0 + jl;
                    }
                }
            }
        }
        s_pm[g][l] = m;
        s_key[g][l] = ((unsigned long long)(uint32_t)best << 32) | (uint32_t)(bj + 1);
        __syncthreads();
        if (g == 0) {
            float mm = s_pm[0][l];
            unsigned long long key = s_key[0][l];
#pragma unroll
            for (int u = 1; u < 4; ++u) {
                mm = s_pm[u][l] > mm ? s_pm[u][l] : mm;
                key = s_key[u][l] > key ? s_key[u][l] : key;
            }
            s_m[l] = mm;
            s_key[0][l] = key;
        }
        __syncthreads();
        const float mq = s_m[l];
        // ---- pass 2
        float acc[4][CPT], den[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            den[q] = exp2_fp32(-s_m[4 * qq + q]);
#pragma unroll
            for (int c = 0; c < CPT; ++c) acc[q][c] = 0.0f;
        }
        for (int kt = 0; kt < nkt; ++kt) {
            const int j0 = kt * KT;
            __syncthreads();
            stage_keys(j0);
            stage_rows<T, R>(s_sk, sk, row0, a.H, KT, n, [&](int y) { return j0 + y; }, tid);
            const bool fin =
                stage_rows<T, DV>(s_v, v, row0, a.H, KT, n, [&](int y) { return j0 + y; }, tid);
            dense_lengths<KT>(s_qlab, s_rst, s_klab, s_L, i0, j0, nq, n, bstrip, tid);
            __syncthreads();
            // phase A: lane = query l, keys g*KG .. g*KG + KG - 1
#pragma unroll 2
            for (int u = 0; u < KG; ++u) {
                const int jl = g * KG + u;
                const int L = s_L[l * KS + jl];
                const bool valid = L > 0;
                const float p = valid ? exp2_fp32(lut[L] - mq) : 0.0f;
                float skr[R];
                lds_vec<R>(&s_sk[jl * R], skr);
                float s = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
                s_c[jl * 64 + l] = valid ? p * s : 0.0f;
                s_p[jl * 64 + l] = p;
            }
            __syncthreads();
            // phase B: lanes = 4 queries x CPT columns, keys ascending
            auto fold = [&](auto safe) {
                for (int jl = 0; jl < KT; ++jl) {
                    float c4[4], vv[CPT];
                    lds4(&s_c[jl * 64 + 4 * qq], c4);
                    lds_vec<CPT>(&s_v[jl * DV + cg * CPT], vv);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (decltype(safe)::value && s_L[(4 * qq + q) * KS + jl] == 0) continue;
#pragma unroll
                        for (int c = 0; c < CPT; ++c)
                            acc[q][c] = __builtin_fmaf(c4[q], vv[c], acc[q][c]);
                    }
                    if (cg == 0) {
                        float p4[4];
                        lds4(&s_p[jl * 64 + 4 * qq], p4);
#pragma unroll
                        for (int q = 0; q < 4; ++q) den[q] = den[q] + p4[q];
                    }
                }
            };
            if (fin) fold(std::integral_constant<bool, false>{});
            else fold(std::integral_constant<bool, true>{});
        }
        if (cg == 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) s_den[4 * qq + q] = den[q];
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int il = 4 * qq + q;
            if (il >= nq) continue;
            const float dd = s_den[il];
            float o[CPT];
#pragma unroll
            for (int c = 0; c < CPT; ++c) o[c] = acc[q][c] / dd;
            store_out<T>(a.out, a.out_dtype, (row0 + (long)(i0 + il) * a.H) * DV + cg * CPT, o,
                         CPT);
        }
        if (tid < nq) {
            const float dd = s_den[tid];
            a.lse2[so + i0 + tid] = s_m[tid] + log2_fp32(dd);
            const unsigned long long key = s_key[0][tid];
            if (a.lmax) a.lmax[so + i0 + tid] = (int)(key >> 32);
            if (a.jarg) a.jarg[so + i0 + tid] = (int)(uint32_t)(key & 0xffffffffu) - 1;
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward, query rows (dSQ, rowtau): workgroup per (dense row, 64-query strip).
template <typename T, int R, int DV>
__global__ __launch_bounds__(DENSE_THREADS) void dense_rows_kernel(PathArgs a) {
    constexpr int KT = DK, KS = KT + 1, KG = KT / 4;
    constexpr int RPT = R >= 4 ? R / 4 : 1;  // readout rows per thread in phase B
    __shared__ int s_qlab[64], s_rst[64], s_klab[KT + 64];
    __shared__ int s_L[64 * KS];
    __shared__ __attribute__((aligned(16))) float s_sk[KT * R];
    __shared__ __attribute__((aligned(16))) float s_v[KT * DV];
    __shared__ __attribute__((aligned(16))) float s_pe[KT * 64];
    __shared__ __attribute__((aligned(16))) float s_pse[KT * 64];
    __shared__ __attribute__((aligned(16))) float s_pp[KT * 64];
    __shared__ __attribute__((aligned(16))) float s_gg[KT * 64];
    __shared__ float s_red[4][64];
    const int tid = (int)threadIdx.x, l = tid & 63, g = tid >> 6;
    const int n = a.n, Q = (n + 63) >> 6;
    const int cnt = __builtin_amdgcn_readfirstlane(*a.o.dcount);
    const long items = (long)cnt * Q;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long x = blockIdx.x; x < items; x += gridDim.x) {
        const DenseItem it = dense_item(a, x, cnt, Q, true);
        const int bh = it.bh, qs = it.strip;
        if (!a.hard[bh]) continue;
        const int b = bh / a.H, h = bh - b * a.H;
        const long so = (long)bh * n, row0 = (long)b * n * a.H + h;
        const int i0 = qs * 64, nq = n - i0 < 64 ? n - i0 : 64;
        const uint16_t* bstrip = dense_strip(a, bh, qs);
        const float* lut = a.lut + (long)h * a.lut_stride;
        const float* glut = a.dlut + (long)h * a.lut_stride;
        const int nkt = (i0 + nq + KT - 1) / KT;
        __syncthreads();
        if (tid < 64) {
            s_qlab[tid] = tid < nq ? a.iq[so + i0 + tid] : 0;
            s_rst[tid] = tid < nq ? dense_reset(a, so, i0 + tid) : 0;
        }
        const int il_me = l < nq ? l : 0;
        const int i = i0 + il_me;
        float sqr[R], dor[DV];
        load_row<T, R>(sq + (row0 + (long)i * a.H) * R, sqr);
        load_row<T, DV>(dout + (row0 + (long)i * a.H) * DV, dor);
        const float l2 = a.lse2[so + i];
        const float cc = glut[i - doc_start(a, i) + 1];
        float dq[RPT], chain = 0.0f;  // chain: u (g 0), vv (1), w (2), z (3)
#pragma unroll
        for (int x2 = 0; x2 < RPT; ++x2) dq[x2] = 0.0f;
        const int r0 = g * RPT;
        for (int kt = 0; kt < nkt; ++kt) {
            const int j0 = kt * KT;
            __syncthreads();
            if (tid < KT + 64) {
                const int j = j0 - 64 + tid;
                s_klab[tid] = (j >= 0 && j < n) ? a.ik[so + j] : 0;
            }
            const bool fin = stage_rows<T, R>(s_sk, sk, row0, a.H, KT, n,
                                              [&](int y) { return j0 + y; }, tid);
            stage_rows<T, DV>(s_v, v, row0, a.H, KT, n, [&](int y) { return j0 + y; }, tid);
            dense_lengths<KT>(s_qlab, s_rst, s_klab, s_L, i0, j0, nq, n, bstrip, tid);
            __syncthreads();
            // phase A: lane = query l, keys g*KG ..
#pragma unroll 1
            for (int u = 0; u < KG; ++u) {
                const int jl = g * KG + u;
                const int L = s_L[l * KS + jl];
                const bool valid = L > 0;
                const float p = valid ? exp2_fp32(lut[L] - l2) : 0.0f;
                float s = 0.0f, e = 0.0f;
                {
                    float skr[R];
                    lds_vec<R>(&s_sk[jl * R], skr);
#pragma unroll
                    for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqr[r], skr[r], s);
                }
#pragma unroll
                for (int d0 = 0; d0 < DV; d0 += 16) {
                    float vr[16];
                    lds_vec<16>(&s_v[jl * DV + d0], vr);
#pragma unroll
                    for (int d = 0; d < 16; ++d) e = __builtin_fmaf(dor[d0 + d], vr[d], e);
                }
                const float ps = p * s, pe = p * e, pse = ps * e;
                const float gg = valid ? glut[L] - cc : 0.0f;
                s_pe[jl * 64 + l] = valid ? pe : 0.0f;
                s_pse[jl * 64 + l] = valid ? pse : 0.0f;
                s_pp[jl * 64 + l] = p;
                s_gg[jl * 64 + l] = gg;
            }
            __syncthreads();
            // phase B: lane = query l; g: readout rows r0.., and one of the four chains
            auto fold = [&](auto safe) {
                for (int jl = 0; jl < KT; ++jl) {
                    if (decltype(safe)::value && s_L[l * KS + jl] == 0) continue;
                    const float pe = s_pe[jl * 64 + l];
                    if (r0 < R) {
                        float skr[RPT];
                        lds_vec<RPT>(&s_sk[jl * R + r0], skr);
#pragma unroll
                        for (int x2 = 0; x2 < RPT; ++x2) dq[x2] = __builtin_fmaf(pe, skr[x2], dq[x2]);
                    }
                    if (g == 0) chain = chain + s_pse[jl * 64 + l];
                    else if (g == 1) chain = __builtin_fmaf(s_pp[jl * 64 + l], s_gg[jl * 64 + l], chain);
                    else if (g == 2) chain = __builtin_fmaf(s_pse[jl * 64 + l], s_gg[jl * 64 + l], chain);
                    else chain = chain + s_pp[jl * 64 + l];
                }
            };
            if (fin) fold(std::integral_constant<bool, false>{});
            else fold(std::integral_constant<bool, true>{});
        }
        if (l < nq && r0 < R) {
            float* o = a.dsq + (row0 + (long)(i0 + l) * a.H) * R + r0;
#pragma unroll
            for (int x2 = 0; x2 < RPT; ++x2) o[x2] = dq[x2];
        }
        s_red[g][l] = chain;
        __syncthreads();
        if (g == 0 && l < nq) {
            const float u = s_red[0][l], vv = s_red[1][l], w = s_red[2][l], z = s_red[3][l];
            const float f = exp2_fp32(-l2);
            const float mass = z + f;
            const float mean = __builtin_fmaf(-f, cc, vv) / mass;
            a.rowtau[so + i0 + l] = __builtin_fmaf(-u, mean, w) / mass;
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward, keys (dSK, dV): workgroup per (dense row, strip of DK keys), 64-query tiles
// ascending from the tile holding the strip's first key.
template <typename T, int R, int DV>
__global__ __launch_bounds__(DENSE_THREADS) void dense_keys_kernel(PathArgs a) {
    constexpr int KT = DK, KS = KT + 1, QG = 64 / 8;
    constexpr int RB = R >= 8 ? R / 8 : 1;   // dSK rows per thread (8 row groups)
    constexpr int C2 = DV / 32;              // dV columns per thread (32 column groups)
    __shared__ int s_qlab[64], s_rst[64], s_klab[KT + 64];
    __shared__ int s_L[64 * KS];
    __shared__ __attribute__((aligned(16))) float s_sq[64 * R];
    __shared__ __attribute__((aligned(16))) float s_do[64 * DV];
    __shared__ __attribute__((aligned(16))) float s_pe[64 * KT];
    __shared__ __attribute__((aligned(16))) float s_ps[64 * KT];
    __shared__ float s_l2[64];
    const int tid = (int)threadIdx.x;
    const int kl = tid & 31, g8 = tid >> 5;     // phase A: key kl, queries g8*QG ..
    const int kq = tid & 7, cgv = tid >> 3;     // phase B dV: keys 4kq.., columns cgv*C2 ..
    const int n = a.n, S = (n + KT - 1) / KT;
    const int cnt = __builtin_amdgcn_readfirstlane(*a.o.dcount);
    const long items = (long)cnt * S;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long x = blockIdx.x; x < items; x += gridDim.x) {
        const DenseItem it = dense_item(a, x, cnt, S, false);
        const int bh = it.bh, ks = it.strip;
        if (!a.hard[bh]) continue;
        const int b = bh / a.H, h = bh - b * a.H;
        const long so = (long)bh * n, row0 = (long)b * n * a.H + h;
        const int j0 = ks * KT, nk = n - j0 < KT ? n - j0 : KT;
        const float* lut = a.lut + (long)h * a.lut_stride;
        const int jme = j0 + (kl < nk ? kl : 0);
        float skr[R], vr[DV];
        load_row<T, R>(sk + (row0 + (long)jme * a.H) * R, skr);
        load_row<T, DV>(v + (row0 + (long)jme * a.H) * DV, vr);
        float dk[RB], dv[4][C2];
#pragma unroll
        for (int x2 = 0; x2 < RB; ++x2) dk[x2] = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int c = 0; c < C2; ++c) dv[q][c] = 0.0f;
        const int rk0 = g8 * RB;
        __syncthreads();
        if (tid < KT + 64) {
            const int j = j0 - 64 + tid;
            s_klab[tid] = (j >= 0 && j < n) ? a.ik[so + j] : 0;
        }
        for (int qt = j0 / 64; qt * 64 < n; ++qt) {
            const int i0 = qt * 64, nq = n - i0 < 64 ? n - i0 : 64;
            __syncthreads();
            if (tid < 64) {
                s_qlab[tid] = tid < nq ? a.iq[so + i0 + tid] : 0;
                s_rst[tid] = tid < nq ? dense_reset(a, so, i0 + tid) : 0;
                s_l2[tid] = tid < nq ? a.lse2[so + i0 + tid] : 0.0f;
            }
            const bool f1 = stage_rows<T, R>(s_sq, sq, row0, a.H, 64, n,
                                             [&](int y) { return i0 + y; }, tid);
            const bool f2 = stage_rows<T, DV>(s_do, dout, row0, a.H, 64, n,
                                              [&](int y) { return i0 + y; }, tid);
            dense_lengths<KT>(s_qlab, s_rst, s_klab, s_L, i0, j0, nq, n, dense_strip(a, bh, qt),
                              tid);
            __syncthreads();
            // phase A: lane = key kl, queries g8*QG ..
#pragma unroll 1
            for (int u = 0; u < QG; ++u) {
                const int il = g8 * QG + u;
                const int L = s_L[il * KS + kl];
                const bool valid = L > 0;
                const float p = valid ? exp2_fp32(lut[L] - s_l2[il]) : 0.0f;
                float s = 0.0f, e = 0.0f;
                {
                    float sqv[R];
                    lds_vec<R>(&s_sq[il * R], sqv);
#pragma unroll
                    for (int r = 0; r < R; ++r) s = __builtin_fmaf(sqv[r], skr[r], s);
                }
#pragma unroll
                for (int d0 = 0; d0 < DV; d0 += 16) {
                    float dd[16];
                    lds_vec<16>(&s_do[il * DV + d0], dd);
#pragma unroll
                    for (int d = 0; d < 16; ++d) e = __builtin_fmaf(dd[d], vr[d0 + d], e);
                }
                s_pe[il * KT + kl] = valid ? p * e : 0.0f;
                s_ps[il * KT + kl] = valid ? p * s : 0.0f;
            }
            __syncthreads();
            // phase B: queries ascending
            auto fold = [&](auto safe) {
                for (int il = 0; il < 64; ++il) {
                    // dSK: key kl, rows rk0 ..
                    if (rk0 < R && !(decltype(safe)::value && s_L[il * KS + kl] == 0)) {
                        const float pe = s_pe[il * KT + kl];
                        float sqv[RB];
                        lds_vec<RB>(&s_sq[il * R + rk0], sqv);
#pragma unroll
                        for (int x2 = 0; x2 < RB; ++x2) dk[x2] = __builtin_fmaf(pe, sqv[x2], dk[x2]);
                    }
                    // dV: keys 4kq .. 4kq+3, columns cgv*C2 ..
                    float ps4[4], dd[C2];
                    lds4(&s_ps[il * KT + 4 * kq], ps4);
                    lds_vec<C2>(&s_do[il * DV + cgv * C2], dd);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (decltype(safe)::value && s_L[il * KS + 4 * kq + q] == 0) continue;
#pragma unroll
                        for (int c = 0; c < C2; ++c) dv[q][c] = __builtin_fmaf(ps4[q], dd[c], dv[q][c]);
                    }
                }
            };
            if (f1 && f2) fold(std::integral_constant<bool, false>{});
            else fold(std::integral_constant<bool, true>{});
        }
        if (kl < nk && rk0 < R) {
            float* o = a.dsk + (row0 + (long)(j0 + kl) * a.H) * R + rk0;
#pragma unroll
            for (int x2 = 0; x2 < RB; ++x2) o[x2] = dk[x2];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int jl = 4 * kq + q;
            if (jl >= nk) continue;
            float* o = a.dv + (row0 + (long)(j0 + jl) * a.H) * DV + cgv * C2;
#pragma unroll
            for (int c = 0; c < C2; ++c) o[c] = dv[q][c];
        }
    }
}

// ---------------------------------------------------------------------------------------
hipError_t launch_dense_classify(const int32_t* iq, const int32_t* ik, long BH, int n,
                                 int cls_n, int32_t* dflag, unsigned long long* dcost,
                                 hipStream_t s) {
    const int cn = cls_n > 0 && cls_n < n ? cls_n : n;
    hipLaunchKernelGGL(dense_classify_kernel, dim3((unsigned)BH), dim3(256), 0, s, iq, ik, n, cn,
                       dflag, dcost);
    return hipGetLastError();
}

hipError_t launch_dense_prepare(const PathArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(dense_mode_kernel, dim3(1), dim3(1024), 0, s, a.o.dflag, a.o.dcost,
                       a.B * a.H, a.n, a.o.dlist, a.o.dcount);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.n > DENSE_MAX_N || a.n <= 64) return e;
    hipLaunchKernelGGL(dense_bound_kernel, dim3(DENSE_GRID), dim3(256), 0, s, a);
    return hipGetLastError();
}

#define DISM_DENSE_LAUNCHER(NAME, KERNEL)                                                     \
    template <typename T, int R, int DV>                                                      \
    static hipError_t NAME##_go(const PathArgs& a, hipStream_t s) {                           \
        hipLaunchKernelGGL((KERNEL<T, R, DV>), dim3(DENSE_GRID), dim3(DENSE_THREADS), 0, s,   \
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
        if (a.n > DENSE_MAX_N) return hipSuccess;                                             \
        if (dtype == DTYPE_BF16) return NAME##_r<bf16_t>(a, R, DV, s);                        \
        if (dtype == DTYPE_F32) return NAME##_r<float>(a, R, DV, s);                          \
        return hipErrorInvalidValue;                                                          \
    }

DISM_DENSE_LAUNCHER(dense_forward, dense_forward_kernel)
DISM_DENSE_LAUNCHER(dense_rows, dense_rows_kernel)
DISM_DENSE_LAUNCHER(dense_keys, dense_keys_kernel)

}  // namespace dism
