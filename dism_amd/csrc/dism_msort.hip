// dism_msort.hip -- multi-block stable radix sort of the global-memory prepare, for rows the
// LDS-resident prepare cannot hold (N > PREP_N, packed layouts).
//
// sort_kernel gives one 1024-thread workgroup to each (row, role): a long single sequence has
// few rows (B*H = 16 for one 64K-token sequence of 16 heads), so most CUs idle while the passes
// run one after another.
// Here every row is split into S segments of one 256-thread workgroup each, and every LSD pass
// is two launches:
//   hist:    workgroup (row, s) counts the digits of its segment -> mcount[row][digit][s];
//   scatter: workgroup (row, s) derives the start of each digit run of its segment from the
//            count table (runs of earlier digits anywhere, then the same digit in earlier
//            segments), ranks its elements in order (per-wave digit counts, lane masks built
//            with LDS atomic ORs), chunk by chunk into digit order in LDS, and writes each
//            chunk out with the elements of one digit at consecutive positions.
// Both are stable, so the result equals sort_kernel's (same digits, same pass order, same
// outputs).  The digits used by a row are only known on the device: msort_mask_kernel
// records the label bits each row uses, every pass up to the most a row can need is
// launched, and passes beyond a row's digit count exit at once.
#include "dism_path.h"

DISM_TU_LAYOUT(msort)

namespace dism {

constexpr int MS_THREADS = 256;
constexpr int MS_WAVES = MS_THREADS / 64;
constexpr int MS_RADIX = 256;
constexpr int MS_U = 8;  // elements per lane loaded together

// Label bits used by each (b,h) row, in MS_PARTS partial masks (chunk c of the row's
// positions, query and key labels): mdig[bh*MS_PARTS + c]; msort_digits_kernel ORs them into
// the row's digits, the bytes with any bit set.  grid (B*H, MS_PARTS).
constexpr int MS_PARTS = 32;
__global__ __launch_bounds__(MS_THREADS) void msort_mask_kernel(SortArgs a) {
    __shared__ uint32_t s_mask;
    const int bh = blockIdx.x, c = blockIdx.y, tid = threadIdx.x, n = a.n;
    const long off = (long)bh * n;
    const int per = (n + MS_PARTS - 1) / MS_PARTS;
    const int p0 = c * per, p1 = p0 + per < n ? p0 + per : n;
    if (tid == 0) s_mask = 0;
    __syncthreads();
    uint32_t m = 0;
    for (int p = p0 + tid; p < p1; p += MS_THREADS)
        m |= (uint32_t)a.lab[0][off + p] | (uint32_t)a.lab[1][off + p];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m |= (uint32_t)__shfl_xor((int)m, o);
    if ((tid & 63) == 0) atomicOr(&s_mask, m);
    __syncthreads();
    if (tid == 0) a.o.mdig[(long)bh * MS_PARTS + c] = (int)s_mask;
}

// The row's digits from its partial masks: mdig[B*H*MS_PARTS + bh*8] = count, then the byte
// indices of the digits packed one per byte, low first.  grid (B*H), one wave.
__global__ __launch_bounds__(64) void msort_digits_kernel(SortArgs a) {
    const int bh = blockIdx.x, lane = threadIdx.x;
    uint32_t m = lane < MS_PARTS ? (uint32_t)a.o.mdig[(long)bh * MS_PARTS + lane] : 0u;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m |= (uint32_t)__shfl_xor((int)m, o);
    if (lane == 0) {
        int32_t* h = a.o.mdig + a.BH * MS_PARTS + (long)bh * 8;
        int nd = 0;
        uint32_t packed = 0;
        for (int d = 0; d < 4; ++d)
            if ((m >> (8 * d)) & 255u) packed |= (uint32_t)d << (8 * nd++);
        h[0] = nd;
        h[1] = (int)packed;
    }
}

// the row's digits: count, and the byte index of digit k (low first) in byte k of packed
struct MsDigits {
    int nd;
    uint32_t packed;
    __device__ int byte(int k) const { return (int)((packed >> (8 * k)) & 255u); }
};
__device__ __forceinline__ MsDigits ms_digits(const SortArgs& a, int bh) {
    const int32_t* h = a.o.mdig + a.BH * MS_PARTS + (long)bh * 8;
    MsDigits g;
    g.nd = h[0];
    g.packed = (uint32_t)h[1];
    return g;
}

// What one pass of one row sorts.  kind 0: the combined order of the 2N entries e = 2p + s
// (key: the entry's label); kind 1: the bigram order of one side's N positions (passes
// 0..nd-1 by the label, nd..2nd-1 by the predecessor's label).
struct MsRow {
    int m;                      // elements
    int nd, pass, passes;       // digit count, this pass, passes of the row
    int shift;                  // bit shift of this pass's digit
    int top_shift;              // bit shift of the row's top digit
    bool use_prev;              // kind 1: key is the predecessor's label
    const int32_t* lq;
    const int32_t* lk;
    const int32_t* lab;         // kind 1: this side's labels
    const int32_t* in;          // null: identity
    int32_t* out;
    int32_t* lab_out;           // last pass: label (kind 0) / label (kind 1)
    int32_t* plab_out;          // last pass, kind 1: predecessor's label
    int32_t* table;             // last pass: digit run starts [257]
};

__device__ __forceinline__ bool ms_row(const SortArgs& a, int kind, int row, int pass, MsRow& r) {
    const int n = a.n;
    const int bh = kind == 0 ? row : row >> 1, side = kind == 0 ? 0 : row & 1;
    const long off = (long)bh * n;
    const MsDigits dg = ms_digits(a, bh);
    r.nd = dg.nd;
    r.passes = kind == 0 ? r.nd : 2 * r.nd;
    r.pass = pass;
    if (pass >= (r.passes > 0 ? r.passes : 1)) return false;  // nd == 0: one identity pass
    r.lq = a.lab[0] + off;
    r.lk = a.lab[1] + off;
    const int k = r.nd ? (pass < r.nd ? pass : pass - r.nd) : 0;
    r.shift = r.nd ? 8 * dg.byte(k) : 0;
    r.top_shift = r.nd ? 8 * dg.byte(r.nd - 1) : 0;
    r.use_prev = kind == 1 && pass >= r.nd;
    const bool last = pass == (r.passes > 0 ? r.passes : 1) - 1;
    // ping-pong so that the last pass writes the order itself
    int32_t* fin;
    int32_t* tmp;
    if (kind == 0) {
        r.m = 2 * n;
        r.lab = nullptr;
        fin = a.o.corder + 2 * off;
        tmp = a.tmp[0] + 2 * off;
        r.lab_out = last ? a.o.clab + 2 * off : nullptr;
        r.plab_out = nullptr;
        r.table = last ? a.o.ctab + (long)bh * (MS_RADIX + 1) : nullptr;
    } else {
        r.m = n;
        r.lab = side ? r.lk : r.lq;
        fin = a.o.bpos[side] + off;
        tmp = a.tmp[side + 1] + off;
        r.lab_out = last ? a.o.blab[side] + off : nullptr;
        r.plab_out = last ? a.o.bplab[side] + off : nullptr;
        r.table = last ? a.o.btab[side] + (long)bh * (MS_RADIX + 1) : nullptr;
    }
    const int np = r.passes > 0 ? r.passes : 1;
    r.out = ((np - 1 - pass) & 1) ? tmp : fin;
    r.in = pass == 0 ? nullptr : (((np - pass) & 1) ? tmp : fin);
    return true;
}

// element x of the pass: value (entry or position), its digit, and its output labels
__device__ __forceinline__ void ms_elem(const MsRow& r, int kind, int x, int& v, int& dig,
                                        int& lab1, int& lab2) {
    v = r.in ? r.in[x] : x;
    uint32_t key;
    if (kind == 0) {
        key = (uint32_t)((v & 1) ? r.lq[v >> 1] : r.lk[v >> 1]);
        lab1 = (int)key;
        lab2 = 0;
    } else {
        const uint32_t cur = (uint32_t)r.lab[v];
        const uint32_t prev = v > 0 ? (uint32_t)r.lab[v - 1] : 0u;
        key = r.use_prev ? prev : cur;
        lab1 = (int)cur;
        lab2 = (int)prev;
    }
    dig = r.nd ? (int)((key >> r.shift) & 255u) : 0;
}

struct MsGrid {
    int S, seg, beg, end;
};
__device__ __forceinline__ MsGrid ms_grid(int m, int S, int s) {
    MsGrid g;
    g.S = S;
    g.seg = ((m + S - 1) / S + 63) / 64 * 64;
    g.beg = s * g.seg < m ? s * g.seg : m;
    g.end = g.beg + g.seg < m ? g.beg + g.seg : m;
    return g;
}

// grid (rows, S): digit counts of segment s -> counts[row][digit][s]
__global__ __launch_bounds__(MS_THREADS) void msort_hist_kernel(SortArgs a, int kind, int pass,
                                                                int S, int32_t* counts) {
    __shared__ int s_cnt[MS_RADIX];
    const int row = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
    MsRow r;
    if (!ms_row(a, kind, row, pass, r)) return;
    if (pass == 0 && s == 0 && (kind == 0 || (row & 1) == 0)) {
        // the row's mode (global-memory prepare), shift (top digit) and one-byte flag; the
        // bigram half also clears the class counts the plan appends to
        const int bh = kind == 0 ? row : row >> 1;
        if (tid == 0) {
            a.o.mode[bh] = 0;
            a.o.shift[bh] = r.nd ? r.top_shift : 0;
            a.o.onebyte[bh] = r.nd <= 1 ? 1 : 0;
        }
        if (kind == 1 && tid < 8) a.o.bhcount[tid >> 2][(long)bh * 4 + (tid & 3)] = 0;
    }
    const MsGrid g = ms_grid(r.m, S, s);
    s_cnt[tid] = 0;
    __syncthreads();
    for (int x0 = g.beg; x0 < g.end; x0 += MS_THREADS * MS_U) {
        int dig[MS_U];
#pragma unroll
        for (int u = 0; u < MS_U; ++u) {  // all loads of the batch in flight together
            const int x = x0 + u * MS_THREADS + tid;
            int v, l1, l2;
            ms_elem(r, kind, x < g.end ? x : g.end - 1, v, dig[u], l1, l2);
        }
#pragma unroll
        for (int u = 0; u < MS_U; ++u)
            if (x0 + u * MS_THREADS + tid < g.end) atomicAdd(&s_cnt[dig[u]], 1);
    }
    __syncthreads();
    counts[((long)row * MS_RADIX + tid) * S + s] = s_cnt[tid];
}

// grid (rows, S): stable scatter of segment s, in chunks of MS_CHUNK elements staged in LDS:
// a chunk is ranked in order (per-wave digit counts, lane masks built with LDS atomic ORs)
// into its digit-sorted order in LDS, then written out by consecutive threads, so that the
// elements of one digit go to consecutive output positions (runs of about MS_CHUNK / 256
// elements instead of single 4-byte stores).
constexpr int MS_CHUNK = MS_THREADS * MS_U;  // 2048: 512 elements per wave
__global__ __launch_bounds__(MS_THREADS) void msort_scatter_kernel(SortArgs a, int kind,
                                                                   int pass, int S,
                                                                   const int32_t* counts) {
    __shared__ int s_scan[MS_RADIX];
    __shared__ int s_wcnt[MS_WAVES][MS_RADIX];
    __shared__ unsigned long long s_mask[MS_WAVES][MS_RADIX];
    __shared__ int s_start[MS_RADIX];   // chunk-local start of each digit's run
    __shared__ int s_base[MS_RADIX];    // output position of each digit's next element
    __shared__ int s_v[MS_CHUNK], s_l1[MS_CHUNK], s_l2[MS_CHUNK];
    __shared__ uint8_t s_d[MS_CHUNK];
    const int row = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    MsRow r;
    if (!ms_row(a, kind, row, pass, r)) return;
    const MsGrid g = ms_grid(r.m, S, s);
    // digit d (thread d): total count and count in earlier segments
    int tot = 0, pre = 0;
    {
        const int32_t* c = counts + ((long)row * MS_RADIX + tid) * S;
        for (int t = 0; t < S; ++t) {
            const int v = c[t];
            tot += v;
            if (t < s) pre += v;
        }
    }
    // exclusive scan over digits (one wave, 4 digits per lane): s_scan[d] = the scan of v[d]
    auto digit_scan = [&](int v) {
        s_scan[tid] = v;
        __syncthreads();
        if (tid < 64) {
            const int v0 = s_scan[4 * tid], v1 = s_scan[4 * tid + 1], v2 = s_scan[4 * tid + 2],
                      v3 = s_scan[4 * tid + 3];
            const int sum = v0 + v1 + v2 + v3;
            int inc = sum;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(inc, o);
                if (lane >= o) inc += t;
            }
            int ex = inc - sum;
            s_scan[4 * tid] = ex;
            ex += v0;
            s_scan[4 * tid + 1] = ex;
            ex += v1;
            s_scan[4 * tid + 2] = ex;
            ex += v2;
            s_scan[4 * tid + 3] = ex;
        }
        __syncthreads();
        const int res = s_scan[tid];
        __syncthreads();
        return res;
    };
    const int run0 = digit_scan(tot);  // start of digit tid's run in the whole row
    if (r.table && s == 0) {
        r.table[tid] = run0;
        if (tid == 0) r.table[MS_RADIX] = r.m;
    }
    s_base[tid] = run0 + pre;
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int c0 = g.beg; c0 < g.end; c0 += MS_CHUNK) {
        const int cn = g.end - c0 < MS_CHUNK ? g.end - c0 : MS_CHUNK;
        // wave w takes elements [wb, we) of the chunk, in order
        const int wb = c0 + wave * (MS_CHUNK / MS_WAVES);
        const int we = wb + MS_CHUNK / MS_WAVES < c0 + cn ? wb + MS_CHUNK / MS_WAVES : c0 + cn;
        for (int w = 0; w < MS_WAVES; ++w) {
            s_wcnt[w][tid] = 0;
            s_mask[w][tid] = 0ull;
        }
        __syncthreads();
        int vv[MS_U], dd[MS_U], c1[MS_U], c2[MS_U];
#pragma unroll
        for (int u = 0; u < MS_U; ++u) {  // all loads of the wave's part in flight together
            const int x = wb + 64 * u + lane;
            ms_elem(r, kind, x < we ? x : (we > wb ? we - 1 : c0), vv[u], dd[u], c1[u], c2[u]);
        }
#pragma unroll
        for (int u = 0; u < MS_U; ++u)
            if (wb + 64 * u + lane < we) atomicAdd(&s_wcnt[wave][dd[u]], 1);
        __syncthreads();
        // digit tid: the chunk's count, its run start in the chunk, each wave's start
        int ctot = 0;
        for (int w = 0; w < MS_WAVES; ++w) ctot += s_wcnt[w][tid];
        const int cstart = digit_scan(ctot);
        s_start[tid] = cstart;
        {
            int run = cstart;
            for (int w = 0; w < MS_WAVES; ++w) {
                const int c = s_wcnt[w][tid];
                s_wcnt[w][tid] = run;
                run += c;
            }
        }
        __syncthreads();
        // rank in order within the wave: chunk-local positions in digit order
#pragma unroll
        for (int u = 0; u < MS_U; ++u) {
            const int x = wb + 64 * u + lane;
            if (x < we) {
                const int dig = dd[u];
                atomicOr(&s_mask[wave][dig], 1ull << lane);
                __builtin_amdgcn_wave_barrier();
                const unsigned long long eq = s_mask[wave][dig];
                const int rank = __popcll(eq & below);
                const int lp = s_wcnt[wave][dig] + rank;
                __builtin_amdgcn_wave_barrier();
                if (rank == 0) {
                    s_wcnt[wave][dig] += __popcll(eq);
                    s_mask[wave][dig] = 0ull;
                }
                __builtin_amdgcn_wave_barrier();
                s_v[lp] = vv[u];
                s_l1[lp] = c1[u];
                s_l2[lp] = c2[u];
                s_d[lp] = (uint8_t)dig;
            }
        }
        __syncthreads();
        // write out: consecutive chunk positions of one digit go to consecutive outputs
        for (int t = tid; t < cn; t += MS_THREADS) {
            const int d = s_d[t];
            const int dst = s_base[d] + (t - s_start[d]);
            r.out[dst] = s_v[t];
            if (r.lab_out) r.lab_out[dst] = s_l1[t];
            if (r.plab_out) r.plab_out[dst] = s_l2[t];
        }
        __syncthreads();
        s_base[tid] += ctot;
        __syncthreads();
    }
}

// segments per row: enough workgroups to fill the device, at least 4096 elements each
static int ms_segments(long rows, int m) {
    long S = (1024 + rows - 1) / rows;
    const long cap = (m + 4095) / 4096;
    if (S > cap) S = cap;
    if (S > MSORT_SEGMENTS) S = MSORT_SEGMENTS;
    return S < 1 ? 1 : (int)S;
}

static hipError_t ms_passes(const SortArgs& a, int kind, hipStream_t st) {
    const long rows = kind == 0 ? a.BH : 2 * a.BH;
    const int m = kind == 0 ? 2 * a.n : a.n;
    const int S = ms_segments(rows, m);
    int32_t* counts = a.o.mcount + (kind == 0 ? 0 : a.BH * MS_RADIX * MSORT_SEGMENTS);
    const int maxp = kind == 0 ? 4 : 8;
    for (int p = 0; p < maxp; ++p) {
        hipLaunchKernelGGL(msort_hist_kernel, dim3((unsigned)rows, (unsigned)S), dim3(MS_THREADS),
                           0, st, a, kind, p, S, counts);
        hipLaunchKernelGGL(msort_scatter_kernel, dim3((unsigned)rows, (unsigned)S),
                           dim3(MS_THREADS), 0, st, a, kind, p, S, (const int32_t*)counts);
    }
    return hipGetLastError();
}

hipError_t launch_msort_labels(const SortArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(msort_mask_kernel, dim3((unsigned)a.BH, MS_PARTS), dim3(MS_THREADS), 0, s,
                       a);
    hipLaunchKernelGGL(msort_digits_kernel, dim3((unsigned)a.BH), dim3(64), 0, s, a);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : ms_passes(a, 0, s);
}

hipError_t launch_msort_pairs(const SortArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(msort_mask_kernel, dim3((unsigned)a.BH, MS_PARTS), dim3(MS_THREADS), 0, s,
                       a);
    hipLaunchKernelGGL(msort_digits_kernel, dim3((unsigned)a.BH), dim3(64), 0, s, a);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? e : ms_passes(a, 1, s);
}

}  // namespace dism
