// dism_dense.hip -- dense rows: hard rows whose labels collide often, computed with the
// direct (pairwise) definition, one wave per 64-row strip.
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
// L[64s - 1, j] (16-bit) of every 64-row query strip s.  A strip's lengths then come from
// 64-bit diagonal masks and its boundary row (diag_length).
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
// Invalid cells (no match, or j > i) contribute exact zeros: accumulators start at +0 and
// are never -0, so +0 terms are exact no-ops -- unless the walked side's row holds a
// non-finite value, for which such cells are skipped explicitly.
#include "dism_path.h"

DISM_TU_LAYOUT(dense)

namespace dism {

constexpr int DENSE_THREADS = 256;
constexpr unsigned DENSE_GRID = 512;   // persistent workgroups of the tile kernels

__device__ __forceinline__ uint32_t label_bucket(int32_t x) {
    return ((uint32_t)x * 0x9E3779B1u) >> 20;
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long x, int m) {
    const int lo = __shfl_xor((int)(uint32_t)x, m), hi = __shfl_xor((int)(uint32_t)(x >> 32), m);
    return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
}

// ---------------------------------------------------------------------------------------
// Classification, one 1024-thread workgroup per (b,h) row, counting the first cn positions (a
// prefill's rows are padded after the real tokens): bucket counts of both sides in LDS (runs
// of equal buckets in a thread's consecutive labels added with one atomic), M = sum over the
// buckets of #queries x #keys, dense when 64 M > cn^2 (rows longer than DENSE_MAX_N never
// are).  With `prefix`, a dense row becomes a prefix row (mode 4) when every bucket holds one
// label and, over the positions 1 .. cn - 1 of both sides, one predecessor label: one LDS
// slot per bucket holding (1 << 32) | label, 0 = empty (dism_prefix.h).
constexpr int CLS_THREADS = 1024;
__global__ __launch_bounds__(CLS_THREADS) void dense_classify_kernel(
    const int32_t* __restrict__ iq, const int32_t* __restrict__ ik, int n, int cn, int prefix,
    int32_t* __restrict__ dflag, unsigned long long* __restrict__ dcost,
    int32_t* __restrict__ runcnt) {
    __shared__ uint32_t s_cnt[2][DENSE_BUCKETS];
    __shared__ unsigned long long s_lab[DENSE_BUCKETS], s_pred[DENSE_BUCKETS];
    __shared__ unsigned long long s_red[CLS_THREADS / 64];
    const long bh = blockIdx.x;
    const int tid = threadIdx.x;
    const int32_t* q = iq + bh * n;
    const int32_t* k = ik + bh * n;
    if (n > DENSE_MAX_N) {
        if (tid == 0) {
            dflag[bh] = 0;
            dcost[bh] = 0ull;
            if (runcnt) runcnt[bh] = 0;
        }
        return;
    }
    for (int x = tid; x < 2 * DENSE_BUCKETS; x += CLS_THREADS) (&s_cnt[0][0])[x] = 0u;
    __syncthreads();
    // a thread's consecutive chunk of positions (runs of one bucket cost one atomic)
    const int per = (cn + CLS_THREADS - 1) / CLS_THREADS;
    const int lo = tid * per, hi = lo + per < cn ? lo + per : cn;
#pragma unroll
    for (int side = 0; side < 2; ++side) {
        const int32_t* lab = side ? k : q;
        if (lo < hi) {
            uint32_t cur = label_bucket(lab[lo]), c = 1;
            for (int x = lo + 1; x < hi; ++x) {
                const uint32_t bk = label_bucket(lab[x]);
                if (bk != cur) {
                    atomicAdd(&s_cnt[side][cur], c);
                    cur = bk;
                    c = 0;
                }
                ++c;
            }
            atomicAdd(&s_cnt[side][cur], c);
        }
    }
    __syncthreads();
    unsigned long long m = 0;
    for (int x = tid; x < DENSE_BUCKETS; x += CLS_THREADS)
        m += (unsigned long long)s_cnt[0][x] * s_cnt[1][x];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m += shfl_xor_u64(m, o);
    if ((tid & 63) == 0) s_red[tid >> 6] = m;
    __syncthreads();
    unsigned long long t = 0;
    for (int w = 0; w < CLS_THREADS / 64; ++w) t += s_red[w];
    const bool dense = t * 64ull > (unsigned long long)cn * (unsigned long long)cn;
    bool pre = false;
    if (dense && prefix) {
        for (int x = tid; x < DENSE_BUCKETS; x += CLS_THREADS) {
            s_lab[x] = 0ull;
            s_pred[x] = 0ull;
        }
        __syncthreads();
        auto put = [](unsigned long long* tab, uint32_t b, unsigned long long tag) {
            unsigned long long cur = tab[b];
            if (cur == 0ull) {
                cur = atomicCAS(&tab[b], 0ull, tag);
                if (cur == 0ull) cur = tag;
            }
            return cur != tag;
        };
        bool bad = false;
        for (int base = 0; base < cn && !bad; base += CLS_THREADS) {
            const int p = base + tid;
            if (p < cn) {
#pragma unroll
                for (int side = 0; side < 2; ++side) {
                    const int32_t* L = side ? k : q;
                    const int32_t lab = L[p];
                    const uint32_t b = label_bucket(lab);
                    bad |= put(s_lab, b, (1ull << 32) | (uint32_t)lab);
                    if (p >= 1) bad |= put(s_pred, b, (1ull << 32) | (uint32_t)L[p - 1]);
                }
            }
            bad = __syncthreads_or(bad);
        }
        pre = !bad;
    }
    if (tid == 0) {
        dflag[bh] = dense ? (pre ? 4 : 1) : 0;
        dcost[bh] = 0ull;  // the walk probe adds to it
        if (runcnt) runcnt[bh] = 0;  // and lists the long runs
    }
}

// Row modes and lists (one workgroup, after the walk probe and the level lists): mode 2 for
// the sparse rows whose walk-cost estimate exceeds cn^2 (cn: the positions the classification
// counted, a prefill's real tokens; the estimate covers only those); the mode-1 rows ascending in
// dlist[0..), the rows of modes 1 and 2 in dlist[BH..), the mode-3 rows in dlist[2 BH..), the
// mode-4 rows in dlist[3 BH..), their counts in dcount[0..3].
__global__ __launch_bounds__(1024) void dense_mode_kernel(int32_t* __restrict__ dflag,
                                                          const unsigned long long* __restrict__ dcost,
                                                          int BH, int n, int cn,
                                                          int32_t* __restrict__ dlist,
                                                          int32_t* __restrict__ dcount) {
    constexpr int NL = 4;
    __shared__ int s_w[NL][16];
    __shared__ int s_base[NL];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const unsigned long long nn = (unsigned long long)cn * (unsigned long long)cn;
    if (tid < NL) s_base[tid] = 0;
    __syncthreads();
    for (int c0 = 0; c0 < BH; c0 += 1024) {
        const int x = c0 + tid;
        int mode = x < BH ? dflag[x] : 0;
        if (x < BH && mode == 0 && n <= DENSE_MAX_N && cn > 64 && dcost[x] > nn) {
            mode = 2;
            dflag[x] = 2;
        }
        const unsigned long long ms[NL] = {__ballot(mode == 1), __ballot(mode == 1 || mode == 2),
                                           __ballot(mode == 3), __ballot(mode == 4)};
        if (lane < NL) s_w[lane][w] = __popcll(ms[lane]);
        __syncthreads();
        int base[NL] = {s_base[0], s_base[1], s_base[2], s_base[3]};
        for (int v = 0; v < w; ++v)
            for (int c = 0; c < NL; ++c) base[c] += s_w[c][v];
        const unsigned long long below = (1ull << lane) - 1ull;
        if (mode == 1) dlist[base[0] + __popcll(ms[0] & below)] = x;
        if (mode == 1 || mode == 2) dlist[BH + base[1] + __popcll(ms[1] & below)] = x;
        if (mode == 3) dlist[2 * BH + base[2] + __popcll(ms[2] & below)] = x;
        if (mode == 4) dlist[3 * BH + base[3] + __popcll(ms[3] & below)] = x;
        __syncthreads();
        if (tid < NL) {
            int t = 0;
            for (int v = 0; v < 16; ++v) t += s_w[tid][v];
            s_base[tid] += t;
        }
        __syncthreads();
    }
    if (tid < NL) dcount[tid] = s_base[tid];
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
// Wave-level tiles.  One 64-lane wave owns one work item -- a 64-row query strip (forward,
// dSQ / rowtau: lane = query row) or a 64-key strip (dSK / dV: lane = key) -- and walks the
// other side in ascending order; waves never synchronise with each other.  The walked side's
// row is the same for every lane at each step, so it is read with scalar loads: the FMAs take
// it as an SGPR operand and the scalar unit unpacks bf16.
//
// Match lengths from diagonal masks: for a diagonal d = i - j crossing a 64-row query strip
// i0 .. i0+63, bit r of its mask is (q[i0+r] == k[i0+r-d]) (one ballot, lanes = rows).  The
// length at strip row r is the run of set bits ending at r: it stops at the last clear bit,
// or at the last query reset at or above r (where the match starts afresh), or else runs into
// the strip's boundary row i0 - 1, whose length dense_bound_kernel stored (the carry).

typedef __attribute__((address_space(4))) const uint32_t cu32_t;

// N consecutive elements of a wave-uniform row as fp32 (scalar loads)
template <typename T, int N>
__device__ __forceinline__ void uniform_row(const T* p, float (&out)[N]) {
    cu32_t* w = (cu32_t*)(const void*)p;
    if constexpr (sizeof(T) == 2) {
        static_assert(N % 2 == 0, "bf16 rows hold an even element count");
#pragma unroll
        for (int c = 0; c < N / 2; ++c) {
            const uint32_t x = w[c];
            out[2 * c] = bf16_lo(x);
            out[2 * c + 1] = bf16_hi(x);
        }
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) out[c] = __uint_as_float(w[c]);
    }
}

// acc[e] = fma(c, row[e], acc[e]) over a wave-uniform row (scalar loads), 32 elements per
// chunk so the unpacked chunk fits the scalar registers; SAFE: only where `valid`
template <typename T, int N, bool SAFE>
__device__ __forceinline__ void fma_uniform_row(const T* p, float c, bool valid, float (&acc)[N]) {
    constexpr int CH = N < 32 ? N : 32;
#pragma unroll
    for (int c0 = 0; c0 < N; c0 += CH) {
        float x[CH];
        uniform_row<T, CH>(p + c0, x);
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            if constexpr (SAFE) acc[c0 + e] = valid ? __builtin_fmaf(c, x[e], acc[c0 + e]) : acc[c0 + e];
            else acc[c0 + e] = __builtin_fmaf(c, x[e], acc[c0 + e]);
        }
    }
}

// s = chain over e of fma(a[e], row[e], s) for a wave-uniform row (scalar loads, chunked)
template <typename T, int N>
__device__ __forceinline__ float dot_uniform_row(const T* p, const float (&a)[N]) {
    constexpr int CH = N < 32 ? N : 32;
    float s = 0.0f;
#pragma unroll
    for (int c0 = 0; c0 < N; c0 += CH) {
        float x[CH];
        uniform_row<T, CH>(p + c0, x);
#pragma unroll
        for (int e = 0; e < CH; ++e) s = __builtin_fmaf(a[c0 + e], x[e], s);
    }
    return s;
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// masks and carries of diagonals, addressed by slot (the caller's diagonal numbering)
struct DiagMasks {
    unsigned long long m[128];
    int c[128];
};

// length at strip row r of a diagonal (mask m, carry c); rm: the strip's reset rows
__device__ __forceinline__ int diag_length(unsigned long long m, int c, int r,
                                           unsigned long long rm) {
    const unsigned long long upto = (2ull << r) - 1ull;  // rows 0 .. r (r = 63: all)
    const unsigned long long z = ~m & upto, rz = rm & upto;
    const int p0 = 63 - __clzll((long long)z);   // last mismatch at or above r, -1 if none
    const int pr = 63 - __clzll((long long)rz);  // last reset at or above r, -1 if none
    const int L = pr > p0 ? r - pr + 1 : (p0 >= 0 ? r - p0 : r + 1 + c);
    return ((m >> r) & 1ull) ? L : 0;
}

// length at (strip row r, diagonal d = i - j) from the ring slot d & 127; 0 for d < 0
__device__ __forceinline__ int strip_length(const DiagMasks& D, int d, int r,
                                            unsigned long long rm) {
    const int slot = d & 127;
    const int L = diag_length(D.m[slot], D.c[slot], r, rm);
    return d >= 0 ? L : 0;
}

// Fill slot (d & 127) for diagonals d in [d_lo, d_hi] (d >= 0) of the strip at i0: lanes are
// the strip's rows (qlab: the lane's query label, qv: the row exists).
__device__ __forceinline__ void fill_diags(DiagMasks& D, const int32_t* __restrict__ k, int n,
                                           int i0, int qlab, bool qv,
                                           const uint16_t* __restrict__ bstrip, int d_lo,
                                           int d_hi, int lane) {
    for (int d = d_lo; d <= d_hi; ++d) {
        const int j = i0 + lane - d;
        const bool in = qv && j >= 0 && j < n;
        const int kv = k[in ? j : 0];
        const unsigned long long m = __ballot(in && kv == qlab);
        const int jc = i0 - 1 - d;
        if (lane == 0) {
            D.m[d & 127] = m;
            D.c[d & 127] = (bstrip && jc >= 0) ? (int)bstrip[jc] : 0;
        }
    }
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

// 1 when every element of row p (N elements of T) is finite
template <typename T, int N>
__device__ __forceinline__ bool row_finite(const T* p) {
    float f[N];
    load_row<T, N>(p, f);
    bool ok = true;
#pragma unroll
    for (int c = 0; c < N; ++c) ok = ok && (__builtin_fabsf(f[c]) <= 3.402823466e38f);
    return ok;
}

template <int N>
__device__ __forceinline__ void store_f32_row(float* o, const float (&x)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int c = 0; c < N / 4; ++c)
            reinterpret_cast<float4*>(o)[c] = make_float4(x[4 * c], x[4 * c + 1], x[4 * c + 2],
                                                          x[4 * c + 3]);
    } else {
#pragma unroll
        for (int c = 0; c < N; ++c) o[c] = x[c];
    }
}

template <int N>
__device__ __forceinline__ void store_row(void* out, int out_dtype, long idx,
                                          const float (&x)[N]) {
    if (out_dtype == DTYPE_F32) {
        store_f32_row<N>(reinterpret_cast<float*>(out) + idx, x);
    } else {
        uint32_t* o = reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(out) + idx);
#pragma unroll
        for (int c = 0; c < N; c += 2)
            o[c / 2] = f32_to_bf16_bits(x[c]) | (f32_to_bf16_bits(x[c + 1]) << 16);
    }
}

constexpr int DKT = 32;  // keys per diagonal refill of the query-strip kernels

// ---------------------------------------------------------------------------------------
// forward: wave per (dense row, 64-query strip); pass 1 the row shift m and the longest
// match, pass 2 the readout, keys ascending.
template <typename T, int R, int DV>
__global__ __launch_bounds__(DENSE_THREADS) void dense_forward_kernel(PathArgs a) {
    __shared__ DiagMasks s_d[DENSE_THREADS / 64];
    const int lane = lane_id(), w = wave_id();
    DiagMasks& D = s_d[w];
    const int n = a.n, Q = (n + 63) >> 6;
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[0]);
    const long items = (long)cnt * Q;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    for (long x = (long)blockIdx.x * (DENSE_THREADS / 64) + w; x < items;
         x += (long)gridDim.x * (DENSE_THREADS / 64)) {
        const DenseItem it = dense_item(a, x, cnt, Q, true);
        const int bh = __builtin_amdgcn_readfirstlane(it.bh);
        const int qs = __builtin_amdgcn_readfirstlane(it.strip);
        if (!a.hard[bh]) continue;
        const int b = bh / a.H, h = bh - b * a.H;
        const long so = (long)bh * n, row0 = (long)b * n * a.H + h;
        const int i0 = qs * 64, nq = n - i0 < 64 ? n - i0 : 64;
        const int i = i0 + lane;
        const bool qv = lane < nq;
        const int32_t* k = a.ik + so;
        const int qlab = qv ? a.iq[so + i] : 0;
        const unsigned long long rm = __ballot(qv && dense_reset(a, so, i));
        const uint16_t* bstrip = dense_strip(a, bh, qs);
        const float* lut = a.lut + (long)h * a.lut_stride;
        const int nk = i0 + nq;  // keys 0 .. nk-1 can pair with the strip
        float sqr[R];
        load_row<T, R>(sq + (row0 + (long)(qv ? i : i0) * a.H) * R, sqr);
        // ---- pass 1: m = max(0, LUT[L]), longest match (ties -> largest key)
        float m = 0.0f;
        int best = 0, bj = -1;
        int filled = i0 + 64;  // lowest diagonal filled so far
        for (int j0 = 0; j0 < nk; j0 += DKT) {
            const int lo = i0 - (j0 + DKT - 1) > 0 ? i0 - (j0 + DKT - 1) : 0;
            const int hi = i0 + 63 - j0 < filled - 1 ? i0 + 63 - j0 : filled - 1;
            fill_diags(D, k, n, i0, qlab, qv, bstrip, lo, hi, lane);
            filled = lo;
            wave_sync_lds();
            const int je = j0 + DKT < nk ? j0 + DKT : nk;
            for (int j = j0; j < je; ++j) {
                const int L = strip_length(D, i - j, lane, rm);
                if (L > 0) {
                    const float lw = lut[L];
                    if (lw > m) m = lw;
                    if (L >= best) {
                        best = L;
                        bj = j;
                    }
                }
            }
            wave_sync_lds();
        }
        // ---- pass 2: den = exp2(-m) + sum p; acc = sum (p s) v, keys ascending
        float den = exp2_fp32(-m), acc[DV];
#pragma unroll
        for (int d = 0; d < DV; ++d) acc[d] = 0.0f;
        filled = i0 + 64;
        for (int j0 = 0; j0 < nk; j0 += DKT) {
            const int lo = i0 - (j0 + DKT - 1) > 0 ? i0 - (j0 + DKT - 1) : 0;
            const int hi = i0 + 63 - j0 < filled - 1 ? i0 + 63 - j0 : filled - 1;
            fill_diags(D, k, n, i0, qlab, qv, bstrip, lo, hi, lane);
            filled = lo;
            const int je = j0 + DKT < nk ? j0 + DKT : nk;
            // keys of this refill whose value rows are all finite (the common case): invalid
            // cells then add exact zeros; otherwise they are skipped explicitly
            const int jf = j0 + (lane < DKT ? lane : 0);
            const unsigned long long fin =
                __ballot(lane < je - j0 && row_finite<T, DV>(v + (row0 + (long)jf * a.H) * DV));
            wave_sync_lds();
            auto keys = [&](auto safe) {
                for (int j = j0; j < je; ++j) {
                    const int L = strip_length(D, i - j, lane, rm);
                    const bool valid = L > 0;
                    const long krow = row0 + (long)__builtin_amdgcn_readfirstlane(j) * a.H;
                    const float s = dot_uniform_row<T, R>(sk + krow * R, sqr);
                    const float p = valid ? exp2_fp32(lut[L] - m) : 0.0f;
                    const float c = valid ? p * s : 0.0f;
                    den = den + p;
                    fma_uniform_row<T, DV, decltype(safe)::value>(v + krow * DV, c, valid, acc);
                }
            };
            // (a tile whose value rows are all finite lets invalid cells add exact zeros)
            if (fin == (je - j0 == 64 ? ~0ull : ((1ull << (je - j0)) - 1ull)))
                keys(std::integral_constant<bool, false>{});
            else
                keys(std::integral_constant<bool, true>{});
            wave_sync_lds();
        }
        if (qv) {
            float o[DV];
#pragma unroll
            for (int e = 0; e < DV; ++e) o[e] = acc[e] / den;
            store_row<DV>(a.out, a.out_dtype, (row0 + (long)i * a.H) * DV, o);
            a.lse2[so + i] = m + log2_fp32(den);
            if (a.lmax) a.lmax[so + i] = best;
            if (a.jarg) a.jarg[so + i] = bj;
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward, query rows (dSQ, rowtau): wave per (dense row, 64-query strip), keys ascending.
template <typename T, int R, int DV>
__global__ __launch_bounds__(DENSE_THREADS) void dense_rows_kernel(PathArgs a) {
    __shared__ DiagMasks s_d[DENSE_THREADS / 64];
    const int lane = lane_id(), w = wave_id();
    DiagMasks& D = s_d[w];
    const int n = a.n, Q = (n + 63) >> 6;
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[0]);
    const long items = (long)cnt * Q;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long x = (long)blockIdx.x * (DENSE_THREADS / 64) + w; x < items;
         x += (long)gridDim.x * (DENSE_THREADS / 64)) {
        const DenseItem it = dense_item(a, x, cnt, Q, true);
        const int bh = __builtin_amdgcn_readfirstlane(it.bh);
        const int qs = __builtin_amdgcn_readfirstlane(it.strip);
        if (!a.hard[bh]) continue;
        const int b = bh / a.H, h = bh - b * a.H;
        const long so = (long)bh * n, row0 = (long)b * n * a.H + h;
        const int i0 = qs * 64, nq = n - i0 < 64 ? n - i0 : 64;
        const int i = i0 + lane;
        const bool qv = lane < nq;
        const int ic = qv ? i : i0;
        const int32_t* k = a.ik + so;
        const int qlab = qv ? a.iq[so + i] : 0;
        const unsigned long long rm = __ballot(qv && dense_reset(a, so, i));
        const uint16_t* bstrip = dense_strip(a, bh, qs);
        const float* lut = a.lut + (long)h * a.lut_stride;
        const float* glut = a.dlut + (long)h * a.lut_stride;
        const int nk = i0 + nq;
        float sqr[R], dor[DV];
        load_row<T, R>(sq + (row0 + (long)ic * a.H) * R, sqr);
        load_row<T, DV>(dout + (row0 + (long)ic * a.H) * DV, dor);
        const float l2 = a.lse2[so + ic];
        const float cc = glut[ic - doc_start(a, ic) + 1];
        float dq[R], u = 0.0f, vv = 0.0f, ww = 0.0f, z = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) dq[r] = 0.0f;
        int filled = i0 + 64;
        for (int j0 = 0; j0 < nk; j0 += DKT) {
            const int lo = i0 - (j0 + DKT - 1) > 0 ? i0 - (j0 + DKT - 1) : 0;
            const int hi = i0 + 63 - j0 < filled - 1 ? i0 + 63 - j0 : filled - 1;
            fill_diags(D, k, n, i0, qlab, qv, bstrip, lo, hi, lane);
            filled = lo;
            const int je = j0 + DKT < nk ? j0 + DKT : nk;
            const int jf = j0 + (lane < DKT ? lane : 0);
            const unsigned long long fin =
                __ballot(lane < je - j0 && row_finite<T, R>(sk + (row0 + (long)jf * a.H) * R));
            wave_sync_lds();
            auto keys = [&](auto safe) {
                for (int j = j0; j < je; ++j) {
                    const int L = strip_length(D, i - j, lane, rm);
                    const bool valid = L > 0;
                    const long krow = row0 + (long)__builtin_amdgcn_readfirstlane(j) * a.H;
                    const float s = dot_uniform_row<T, R>(sk + krow * R, sqr);
                    const float e = dot_uniform_row<T, DV>(v + krow * DV, dor);
                    const float p = valid ? exp2_fp32(lut[L] - l2) : 0.0f;
                    const float ps = p * s, pe = valid ? p * e : 0.0f;
                    const float pse = valid ? ps * e : 0.0f;
                    const float g = valid ? glut[L] - cc : 0.0f;
                    fma_uniform_row<T, R, decltype(safe)::value>(sk + krow * R, pe, valid, dq);
                    u = u + pse;
                    vv = __builtin_fmaf(p, g, vv);
                    ww = __builtin_fmaf(pse, g, ww);
                    z = z + p;
                }
            };
            if (fin == (je - j0 == 64 ? ~0ull : ((1ull << (je - j0)) - 1ull)))
                keys(std::integral_constant<bool, false>{});
            else
                keys(std::integral_constant<bool, true>{});
            wave_sync_lds();
        }
        if (qv) {
            store_f32_row<R>(a.dsq + (row0 + (long)i * a.H) * R, dq);
            const float f = exp2_fp32(-l2);
            const float mass = z + f;
            const float mean = __builtin_fmaf(-f, cc, vv) / mass;
            a.rowtau[so + i] = __builtin_fmaf(-u, mean, ww) / mass;
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward, keys (dSK, dV): wave per (dense row, 64-key strip), lane = key, queries ascending
// from the strip's first key; the masks of each 64-row query strip are rebuilt (lanes =
// rows for the ballots).
template <typename T, int R, int DV>
__global__ __launch_bounds__(DENSE_THREADS) void dense_keys_kernel(PathArgs a) {
    __shared__ DiagMasks s_d[DENSE_THREADS / 64];
    const int lane = lane_id(), w = wave_id();
    DiagMasks& D = s_d[w];
    const int n = a.n, S = (n + 63) >> 6;
    const int cnt = __builtin_amdgcn_readfirstlane(a.o.dcount[0]);
    const long items = (long)cnt * S;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);
    for (long x = (long)blockIdx.x * (DENSE_THREADS / 64) + w; x < items;
         x += (long)gridDim.x * (DENSE_THREADS / 64)) {
        const DenseItem it = dense_item(a, x, cnt, S, false);
        const int bh = __builtin_amdgcn_readfirstlane(it.bh);
        const int ks = __builtin_amdgcn_readfirstlane(it.strip);
        if (!a.hard[bh]) continue;
        const int b = bh / a.H, h = bh - b * a.H;
        const long so = (long)bh * n, row0 = (long)b * n * a.H + h;
        const int j0 = ks * 64, nk = n - j0 < 64 ? n - j0 : 64;
        const int j = j0 + lane;
        const bool kv = lane < nk;
        const int jc = kv ? j : j0;
        const int32_t* k = a.ik + so;
        const float* lut = a.lut + (long)h * a.lut_stride;
        float skr[R], vr[DV];
        load_row<T, R>(sk + (row0 + (long)jc * a.H) * R, skr);
        load_row<T, DV>(v + (row0 + (long)jc * a.H) * DV, vr);
        float dk[R], dvv[DV];
#pragma unroll
        for (int r = 0; r < R; ++r) dk[r] = 0.0f;
#pragma unroll
        for (int e = 0; e < DV; ++e) dvv[e] = 0.0f;
        for (int qt = ks; qt < S; ++qt) {
            const int i0 = qt * 64, nq = n - i0 < 64 ? n - i0 : 64;
            // masks of the diagonals d = i - j in [i0 - j0 - 63, i0 - j0 + 63] at slot
            // d - (i0 - j0 - 63); ballots with lanes = the query strip's rows
            const bool rv = lane < nq;
            const int qlab = rv ? a.iq[so + i0 + lane] : 0;
            const unsigned long long rm = __ballot(rv && dense_reset(a, so, i0 + lane));
            const uint16_t* bstrip = dense_strip(a, bh, qt);
            const int dbase = i0 - j0 - 63;
            for (int t = 0; t < 127; ++t) {
                const int d = dbase + t;
                const int jj = i0 + lane - d;
                const bool in = rv && d >= 0 && jj >= 0 && jj < n;
                const int kk = k[in ? jj : 0];
                const unsigned long long mm = __ballot(in && kk == qlab);
                const int jcar = i0 - 1 - d;
                if (lane == 0) {
                    D.m[t] = mm;
                    D.c[t] = (bstrip && d >= 0 && jcar >= 0) ? (int)bstrip[jcar] : 0;
                }
            }
            // are the strip's sq and dO rows all finite
            const long qrow_l = row0 + (long)(rv ? i0 + lane : i0) * a.H;
            const bool fin_all =
                __ballot(!rv || (row_finite<T, R>(sq + qrow_l * R) &&
                                 row_finite<T, DV>(dout + qrow_l * DV))) == ~0ull;
            wave_sync_lds();
            auto rows = [&](auto safe) {
            constexpr bool SAFE = decltype(safe)::value;
            for (int il = 0; il < nq; ++il) {
                const int i = i0 + il;
                const int t = il - lane + 63;  // slot of d = i - j
                const int L0 = diag_length(D.m[t], D.c[t], il, rm);
                const int L = (i >= j && kv) ? L0 : 0;
                const bool valid = L > 0;
                const long qrow = row0 + (long)__builtin_amdgcn_readfirstlane(i) * a.H;
                const float l2 = a.lse2[so + __builtin_amdgcn_readfirstlane(i)];
                // (fma(a, b, s) = fma(b, a, s): the chains s = sum sq[r] sk[r] and
                // e = sum dO[q] v[q] in the documented order)
                const float s = dot_uniform_row<T, R>(sq + qrow * R, skr);
                const float e = dot_uniform_row<T, DV>(dout + qrow * DV, vr);
                const float p = valid ? exp2_fp32(lut[L] - l2) : 0.0f;
                const float pe = valid ? p * e : 0.0f, ps = valid ? p * s : 0.0f;
                fma_uniform_row<T, R, SAFE>(sq + qrow * R, pe, valid, dk);
                fma_uniform_row<T, DV, SAFE>(dout + qrow * DV, ps, valid, dvv);
            }
            };
            if (fin_all) rows(std::integral_constant<bool, false>{});
            else rows(std::integral_constant<bool, true>{});
            wave_sync_lds();
        }
        if (kv) {
            store_f32_row<R>(a.dsk + (row0 + (long)j * a.H) * R, dk);
            store_f32_row<DV>(a.dv + (row0 + (long)j * a.H) * DV, dvv);
        }
    }
}

// ---------------------------------------------------------------------------------------
hipError_t launch_dense_classify(const int32_t* iq, const int32_t* ik, long BH, int n,
                                 int cls_n, int prefix, int32_t* dflag,
                                 unsigned long long* dcost, int32_t* runcnt, hipStream_t s) {
    const int cn = cls_n > 0 && cls_n < n ? cls_n : n;
    hipLaunchKernelGGL(dense_classify_kernel, dim3((unsigned)BH), dim3(CLS_THREADS), 0, s, iq,
                       ik, n, cn, prefix, dflag, dcost, runcnt);
    return hipGetLastError();
}

hipError_t launch_dense_prepare(const PathArgs& a, hipStream_t s) {
    const hipError_t le = launch_level_prep(a, s);
    if (le != hipSuccess) return le;
    hipLaunchKernelGGL(dense_mode_kernel, dim3(1), dim3(1024), 0, s, a.o.dflag, a.o.dcost,
                       a.B * a.H, a.n, a.cls_n > 0 && a.cls_n < a.n ? a.cls_n : a.n, a.o.dlist,
                       a.o.dcount);
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
