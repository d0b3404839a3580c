// dism_sort.hip -- the position orders every kernel of the hard core works from.
//
// Per (batch, head) row, three 1024-thread workgroups:
//   y = 0  combined label order: the 2N entries e = 2p + s (s = 0 key at position p, s = 1
//          query at position p) stably sorted by their label (unsigned).  Inside a label
//          group the entries are then in position order with a key before the query of the
//          same position, i.e. exactly the merge order of the label scans (a query sees the
//          keys j <= i that precede it).
//   y = 1  bigram order of the queries, y = 2 of the keys: positions stably sorted by
//          (label[p-1], label[p]) with label[-1] := 0 (bigram groups are the candidates for
//          matches of length >= 2, positions ascending inside a group).
// All are least-significant-digit radix sorts with 8-bit digits.  Digits that are zero for
// every label of the row (union of both sides) are skipped -- a stable pass over a constant
// digit is the identity -- so labels below 256 take one pass per key.  Each pass is a stable
// counting sort by 16 waves on contiguous segments: per-wave digit histograms from ballot
// matching, one exclusive scan over (digit, wave), then a scatter with the same ranks.  The
// last pass's digit runs are written out (ctab / btab) together with that digit's shift.
#include "dism_device.h"
#include "dism_launch.h"

DISM_TU_LAYOUT(sort)

namespace dism {

constexpr int SORT_THREADS = 1024;
constexpr int SORT_WAVES = SORT_THREADS / 64;
constexpr int RADIX = 256;
constexpr int UNROLL = 8;

__device__ __forceinline__ unsigned long long match_digit(int dig) {
    // lanes of the wave whose 9-bit value equals this lane's
    unsigned long long eq = ~0ull;
#pragma unroll
    for (int bit = 0; bit < 9; ++bit) {
        const unsigned long long bal = __ballot((dig >> bit) & 1);
        eq &= ((dig >> bit) & 1) ? bal : ~bal;
    }
    return eq;
}

// One stable counting-sort pass over n elements.  Element x of the input is
// in ? in[x] : x; key(v) gives the 32-bit value whose digit (>> shift) & 255 sorts it;
// out1(v) / out2(v) give optional companion values written in output order.
template <typename Key, typename O1, typename O2>
__device__ void sort_pass(int n, const int32_t* in, int32_t* out, int shift, Key key,
                          int32_t* lab_out, O1 out1, int32_t* plab_out, O2 out2, int32_t* table,
                          int (*wcnt)[RADIX], int* scan) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int seg = ((n + SORT_WAVES - 1) / SORT_WAVES + 63) / 64 * 64;
    const int beg = wave * seg;
    const int end = beg + seg < n ? beg + seg : n;
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    // clamped indices: every lane issues its loads unconditionally, UNROLL gathers overlap
    auto element = [&](int x, int& v, int& dig) {
        const int xc = x < end ? x : end - 1;
        v = in ? in[xc] : xc;
        dig = x < end ? (int)((key(v) >> shift) & 255u) : RADIX;
    };

    for (int e = tid; e < SORT_WAVES * RADIX; e += SORT_THREADS) (&wcnt[0][0])[e] = 0;
    __syncthreads();
    if (beg < end) {  // phase 1: per-wave histograms (each wave owns its row of wcnt)
        for (int base0 = beg; base0 < end; base0 += 64 * UNROLL) {
            int vv[UNROLL], dig[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) element(base0 + 64 * u + lane, vv[u], dig[u]);
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const unsigned long long eq = match_digit(dig[u]);
                if (dig[u] < RADIX && __popcll(eq & below) == 0)
                    wcnt[wave][dig[u]] += __popcll(eq);
            }
        }
    }
    __syncthreads();
    // phase 2: exclusive scan in (digit, wave) order -> start of each wave's digit run
    if (tid < RADIX) {
        int tot = 0;
        for (int w = 0; w < SORT_WAVES; ++w) tot += wcnt[w][tid];
        scan[tid] = tot;
    }
    __syncthreads();
    if (tid < 64) {  // one wave scans the 256 totals, 4 per lane
        const int v0 = scan[4 * tid], v1 = scan[4 * tid + 1], v2 = scan[4 * tid + 2],
                  v3 = scan[4 * tid + 3];
        const int sum = v0 + v1 + v2 + v3;
        int inc = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(inc, off);
            if (lane >= off) inc += t;
        }
        int ex = inc - sum;
        scan[4 * tid] = ex;
        ex += v0;
        scan[4 * tid + 1] = ex;
        ex += v1;
        scan[4 * tid + 2] = ex;
        ex += v2;
        scan[4 * tid + 3] = ex;
    }
    __syncthreads();
    if (tid < RADIX) {
        int run = scan[tid];
        for (int w = 0; w < SORT_WAVES; ++w) {
            const int c = wcnt[w][tid];
            wcnt[w][tid] = run;
            run += c;
        }
    }
    __syncthreads();
    if (beg < end) {  // phase 3: scatter (same ranks as phase 1; cursor rows are wave-private)
        for (int base0 = beg; base0 < end; base0 += 64 * UNROLL) {
            int vv[UNROLL], dig[UNROLL], c1[UNROLL], c2[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                element(base0 + 64 * u + lane, vv[u], dig[u]);
                c1[u] = lab_out ? out1(vv[u]) : 0;
                c2[u] = plab_out ? out2(vv[u]) : 0;
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const bool ok = dig[u] < RADIX;
                const unsigned long long eq = match_digit(dig[u]);
                const int rank = __popcll(eq & below);
                int dst = 0;
                if (ok) dst = wcnt[wave][dig[u]] + rank;
                __builtin_amdgcn_wave_barrier();
                if (ok && rank == 0) wcnt[wave][dig[u]] += __popcll(eq);
                if (ok) {
                    out[dst] = vv[u];
                    if (lab_out) lab_out[dst] = c1[u];
                    if (plab_out) plab_out[dst] = c2[u];
                }
            }
        }
    }
    if (table && tid <= RADIX) table[tid] = tid < RADIX ? scan[tid] : n;
    __syncthreads();
}

// One stable counting-sort pass over m elements held in LDS: digit(x) is the 8-bit digit
// of input element x, emit(x, dst) places it.  Per-wave contiguous segments and a scan over
// (digit, wave) as in sort_pass; the histogram takes LDS atomic adds and the ranks inside a
// 64-element group come from per-digit lane masks built with LDS atomic ORs (both
// order-free, so the result is deterministic), instead of bit-by-bit ballot matching.
template <typename Dig, typename Emit>
__device__ void lds_pass(int m, Dig digit, Emit emit, int32_t* table, int (*wcnt)[RADIX],
                         int* scan, unsigned long long (*lmask)[RADIX]) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int seg = ((m + SORT_WAVES - 1) / SORT_WAVES + 63) / 64 * 64;
    const int beg = wave * seg;
    const int end = beg + seg < m ? beg + seg : m;
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int e = tid; e < SORT_WAVES * RADIX; e += SORT_THREADS) {
        (&wcnt[0][0])[e] = 0;
        (&lmask[0][0])[e] = 0ull;
    }
    __syncthreads();
    for (int x = beg + lane; x < end; x += 64) atomicAdd(&wcnt[wave][digit(x)], 1);
    __syncthreads();
    if (tid < RADIX) {
        int tot = 0;
        for (int w = 0; w < SORT_WAVES; ++w) tot += wcnt[w][tid];
        scan[tid] = tot;
    }
    __syncthreads();
    if (tid < 64) {
        const int v0 = scan[4 * tid], v1 = scan[4 * tid + 1], v2 = scan[4 * tid + 2],
                  v3 = scan[4 * tid + 3];
        const int sum = v0 + v1 + v2 + v3;
        int inc = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(inc, off);
            if (lane >= off) inc += t;
        }
        int ex = inc - sum;
        scan[4 * tid] = ex;
        ex += v0;
        scan[4 * tid + 1] = ex;
        ex += v1;
        scan[4 * tid + 2] = ex;
        ex += v2;
        scan[4 * tid + 3] = ex;
    }
    __syncthreads();
    if (tid < RADIX) {
        int run = scan[tid];
        for (int w = 0; w < SORT_WAVES; ++w) {
            const int c = wcnt[w][tid];
            wcnt[w][tid] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int x0 = beg; x0 < end; x0 += 64) {
        const int x = x0 + lane;
        if (x < end) {
            const int dig = digit(x);
            atomicOr(&lmask[wave][dig], 1ull << lane);
            __builtin_amdgcn_wave_barrier();
            const unsigned long long eq = lmask[wave][dig];
            const int rank = __popcll(eq & below);
            const int dst = wcnt[wave][dig] + rank;
            __builtin_amdgcn_wave_barrier();
            if (rank == 0) {
                wcnt[wave][dig] += __popcll(eq);
                lmask[wave][dig] = 0ull;
            }
            __builtin_amdgcn_wave_barrier();
            emit(x, dst);
        }
    }
    if (table && tid <= RADIX) table[tid] = tid < RADIX ? scan[tid] : m;
    __syncthreads();
}

// Combined label order of row bh's 2N entries in global memory (LSD passes over the row's nd
// used label bytes digits[], low first): corder / clab / ctab.  One 1024-thread workgroup;
// wcnt and scan are LDS scratch.
__device__ void label_order_global(const SortArgs& a, int bh, int nd, const int* digits,
                                   int (*wcnt)[RADIX], int* scan) {
    const int n = a.n, tid = threadIdx.x;
    const long off = (long)bh * n;
    const int32_t* __restrict__ lq = a.lab[0] + off;
    const int32_t* __restrict__ lk = a.lab[1] + off;
    const int n2 = 2 * n;
    int32_t* corder = a.o.corder + 2 * off;
    int32_t* clab = a.o.clab + 2 * off;
    int32_t* ctab = a.o.ctab + (long)bh * (RADIX + 1);
    int32_t* tmp = a.tmp[0] + 2 * off;
    auto lab_of = [&](int v) -> uint32_t {
        return (uint32_t)((v & 1) ? lq[v >> 1] : lk[v >> 1]);
    };
    auto lab_out = [&](int v) -> int { return (int)lab_of(v); };
    auto none = [&](int) -> int { return 0; };
    if (nd == 0) {
        for (int x = tid; x < n2; x += SORT_THREADS) {
            corder[x] = x;
            clab[x] = (int)lab_of(x);
        }
        if (tid <= RADIX) ctab[tid] = tid == 0 ? 0 : n2;
        return;
    }
    const int32_t* in = nullptr;
    for (int k = 0; k < nd; ++k) {
        const bool last = k == nd - 1;
        int32_t* out = ((nd - 1 - k) & 1) ? tmp : corder;
        sort_pass(n2, in, out, 8 * digits[k], lab_of, last ? clab : nullptr, lab_out,
                  nullptr, none, last ? ctab : nullptr, wcnt, scan);
        in = out;
    }
}

// grid (BH, 3)
__global__ __launch_bounds__(SORT_THREADS) void sort_kernel(SortArgs a) {
    __shared__ int wcnt[SORT_WAVES][RADIX];
    __shared__ int scan[RADIX];
    __shared__ uint32_t mask;
    const int bh = blockIdx.x, role = (int)blockIdx.y + a.role_base, n = a.n, tid = threadIdx.x;
    const long off = (long)bh * n;
    const int32_t* __restrict__ lq = a.lab[0] + off;
    const int32_t* __restrict__ lk = a.lab[1] + off;

    if (tid == 0) mask = 0;
    __syncthreads();
    uint32_t m = 0;
    for (int x0 = 0; x0 < n; x0 += SORT_THREADS * 4) {
        int32_t v[8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int x = x0 + u * SORT_THREADS + tid;
            const int xc = x < n ? x : n - 1;
            v[2 * u] = lq[xc];
            v[2 * u + 1] = lk[xc];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) m |= (uint32_t)v[u];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m |= (uint32_t)__shfl_xor((int)m, o);
    if ((tid & 63) == 0) atomicOr(&mask, m);
    __syncthreads();
    const uint32_t used = mask;
    int digits[4], nd = 0;
    for (int d = 0; d < 4; ++d)
        if ((used >> (8 * d)) & 255u) digits[nd++] = d;
    // rows with one label byte are prepare_lds_kernel's when it runs (lds_rows): the same
    // test it makes.  Every role writes the row's mode and shift (the same values
    // prepare_lds_kernel writes; the roles may run on different streams); role 1 clears the
    // plan's per-row class counts (the plan appends to them after roles 1 and 2)
    const bool lds = a.lds_rows && nd == 1;
    if (tid == 0) {
        a.o.mode[bh] = lds ? 1 : 0;
        a.o.shift[bh] = nd ? 8 * digits[nd - 1] : 0;
        a.o.onebyte[bh] = nd <= 1 ? 1 : 0;
    }
    if (lds) return;
    if (role == 1 && tid < 8) a.o.bhcount[tid >> 2][(long)bh * 4 + (tid & 3)] = 0;

    if (role == 0) {
        label_order_global(a, bh, nd, digits, wcnt, scan);
        return;
    }

    // ---- bigram order of one side: label digits, then predecessor-label digits
    const int side = role - 1;  // 0 queries, 1 keys
    const int32_t* __restrict__ lab = side ? lk : lq;
    int32_t* bpos = a.o.bpos[side] + off;
    int32_t* blab = a.o.blab[side] + off;
    int32_t* bplab = a.o.bplab[side] + off;
    int32_t* btab = a.o.btab[side] + (long)bh * (RADIX + 1);
    int32_t* tmp = a.tmp[side + 1] + off;
    auto cur = [&](int p) -> uint32_t { return (uint32_t)lab[p]; };
    auto prev = [&](int p) -> uint32_t { return p > 0 ? (uint32_t)lab[p - 1] : 0u; };
    auto cur_i = [&](int p) -> int { return (int)cur(p); };
    auto prev_i = [&](int p) -> int { return (int)prev(p); };
    if (nd == 0) {
        for (int x = tid; x < n; x += SORT_THREADS) {
            bpos[x] = x;
            blab[x] = lab[x];
            bplab[x] = (int)prev(x);
        }
        if (tid <= RADIX) btab[tid] = tid == 0 ? 0 : n;
        return;
    }
    const int passes = 2 * nd;
    const int32_t* in = nullptr;
    for (int k = 0; k < passes; ++k) {
        const bool last = k == passes - 1;
        int32_t* out = ((passes - 1 - k) & 1) ? tmp : bpos;
        if (k < nd)
            sort_pass(n, in, out, 8 * digits[k], cur, nullptr, cur_i, nullptr, prev_i, nullptr,
                      wcnt, scan);
        else
            sort_pass(n, in, out, 8 * digits[k - nd], prev, last ? blab : nullptr, cur_i,
                      last ? bplab : nullptr, prev_i, last ? btab : nullptr, wcnt, scan);
        in = out;
    }
}

// The same counting pass with every wave's elements already in registers: vd[g] holds
// value | digit << 16 of element beg + 64 g + lane (digit RADIX past the end), so the input
// order may be overwritten by emit.  Waves own at most 32 groups (m <= 32768).
template <typename Emit>
__device__ void reg_pass(int m, const uint32_t (&vd)[32], Emit emit, int (*wcnt)[RADIX],
                         int* scan, unsigned long long (*lmask)[RADIX]) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int seg = ((m + SORT_WAVES - 1) / SORT_WAVES + 63) / 64 * 64;
    const int beg = wave * seg;
    const int end = beg + seg < m ? beg + seg : m;
    const int groups = end > beg ? (end - beg + 63) / 64 : 0;
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int e = tid; e < SORT_WAVES * RADIX; e += SORT_THREADS) {
        (&wcnt[0][0])[e] = 0;
        (&lmask[0][0])[e] = 0ull;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < 32; ++g) {
        const int dig = (int)(vd[g] >> 16);
        if (g < groups && dig < RADIX) atomicAdd(&wcnt[wave][dig], 1);
    }
    __syncthreads();
    if (tid < RADIX) {
        int tot = 0;
        for (int w = 0; w < SORT_WAVES; ++w) tot += wcnt[w][tid];
        scan[tid] = tot;
    }
    __syncthreads();
    if (tid < 64) {
        const int v0 = scan[4 * tid], v1 = scan[4 * tid + 1], v2 = scan[4 * tid + 2],
                  v3 = scan[4 * tid + 3];
        const int sum = v0 + v1 + v2 + v3;
        int inc = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(inc, off);
            if (lane >= off) inc += t;
        }
        int ex = inc - sum;
        scan[4 * tid] = ex;
        ex += v0;
        scan[4 * tid + 1] = ex;
        ex += v1;
        scan[4 * tid + 2] = ex;
        ex += v2;
        scan[4 * tid + 3] = ex;
    }
    __syncthreads();
    if (tid < RADIX) {
        int run = scan[tid];
        for (int w = 0; w < SORT_WAVES; ++w) {
            const int c = wcnt[w][tid];
            wcnt[w][tid] = run;
            run += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < 32; ++g) {
        if (g < groups) {
            const int dig = (int)(vd[g] >> 16);
            if (dig < RADIX) {
                atomicOr(&lmask[wave][dig], 1ull << lane);
                __builtin_amdgcn_wave_barrier();
                const unsigned long long eq = lmask[wave][dig];
                const int rank = __popcll(eq & below);
                const int dst = wcnt[wave][dig] + rank;
                __builtin_amdgcn_wave_barrier();
                if (rank == 0) {
                    wcnt[wave][dig] += __popcll(eq);
                    lmask[wave][dig] = 0ull;
                }
                __builtin_amdgcn_wave_barrier();
                emit((int)(vd[g] & 0xFFFFu), dst);
            }
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------------------
// LDS-resident prepare: one (b,h) row per workgroup pair, for N <= PREP_N and labels that
// differ in one byte only (the sign labels of up to 8 binarized features).  Everything the
// pair kernels need is derived from two LDS sorts of the 2N entries e = 2p + s:
//   y = 0  combined label order (as sort_kernel role 0), written out with coalesced stores;
//   y = 1  the same order, then stably by the predecessor's label: the combined BIGRAM order
//          (bigram (label[p-1], label[p]), then e).  In it a bigram group lists keys and
//          queries merged in position order, so for a query row i (p >= 1) its partners are
//          the keys j >= 1 of its group before it, and for a key j (p >= 1) the queries of its
//          group after it.  Prefix counts over the order give each owner its partner range in
//          the side's key / query list (no binary searches), then the owner records, the
//          per-side bigram position lists and the pair counts per query row.
// Each thread owns PREP_E = 2N/1024 consecutive entries of the bigram order (registers);
// block scans combine the threads; outputs are staged in LDS and written coalesced.
constexpr int PREP_E = 2 * PREP_N / SORT_THREADS;  // entries per thread

// Block-wide exclusive scan over the threads, in thread order (rev = false) or reversed
// thread order (rev = true), of an associative op with identity ident.  S is a small
// aggregate of ints; shfl(S, lane) moves one.
template <typename S, typename Op, typename Shfl>
__device__ __forceinline__ S block_exscan(S x, Op op, S ident, Shfl shfl, S* lds, bool rev,
                                          S* total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int vl = rev ? 63 - lane : lane, vw = rev ? SORT_WAVES - 1 - wave : wave;
    S inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const S y = shfl(inc, rev ? lane + off : lane - off);
        if (vl >= off) inc = op(y, inc);
    }
    if (vl == 63) lds[vw] = inc;
    __syncthreads();
    S carry = ident, all = ident;
    for (int w = 0; w < SORT_WAVES; ++w) {
        if (w < vw) carry = op(carry, lds[w]);
        all = op(all, lds[w]);
    }
    S ex = shfl(inc, rev ? lane + 1 : lane - 1);
    if (vl == 0) ex = ident;
    __syncthreads();
    if (total) *total = all;
    return op(carry, ex);
}

struct Seg {     // segmented count: f = a segment start lies inside, v = count after it
    int f, v;
};
struct Cnt4 {
    int x, y, z, w;
};

__global__ __launch_bounds__(SORT_THREADS) void prepare_lds_kernel(SortArgs a) {
    // LDS pool: [dig 2N bytes | rank masks 32 KiB] [order 2N x u16] [digit counters]
    //   after the sorts the first region holds a u16 per entry (partner counts, then the
    //   pair counts per query row) and the order region the per-side position lists.
    // Per-entry u16 arrays are padded by one slot per 32 entries (pad()): threads scan 32
    // consecutive entries, and without the pad every lane of a wave would hit the same banks.
    constexpr int DIG_BYTES = 2 * PREP_N;
    constexpr int MASK_BYTES = SORT_WAVES * RADIX * 8;
    constexpr int PADDED = 2 * PREP_N + 2 * PREP_N / 32;
    constexpr int POOL = DIG_BYTES + MASK_BYTES > 2 * PADDED ? DIG_BYTES + MASK_BYTES : 2 * PADDED;
    __shared__ __attribute__((aligned(16))) unsigned char pool[POOL];
    __shared__ uint16_t s_ord[PADDED];
    __shared__ int wcnt[SORT_WAVES][RADIX];
    __shared__ int scan[RADIX];
    __shared__ uint32_t mask;
    __shared__ Cnt4 s_c4[SORT_WAVES];
    __shared__ Seg s_seg[SORT_WAVES];
    uint8_t* s_dig = pool;
    auto s_mask = reinterpret_cast<unsigned long long (*)[RADIX]>(pool + DIG_BYTES);
    uint16_t* s_cnt = reinterpret_cast<uint16_t*>(pool);  // after the sorts
    auto pad = [](int c) { return c + (c >> 5); };
    const int bh = blockIdx.x, role = (int)blockIdx.y + a.role_base, n = a.n, tid = threadIdx.x;
    const int n2 = 2 * n;
    const long off = (long)bh * n;
    const int32_t* __restrict__ lq = a.lab[0] + off;
    const int32_t* __restrict__ lk = a.lab[1] + off;

    if (tid == 0) mask = 0;
    __syncthreads();
    uint32_t m = 0;
    for (int p = tid; p < n; p += SORT_THREADS) m |= (uint32_t)lq[p] | (uint32_t)lk[p];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m |= (uint32_t)__shfl_xor((int)m, o);
    if ((tid & 63) == 0) atomicOr(&mask, m);
    __syncthreads();
    const uint32_t used = mask;
    int nd = 0, dg = 0;
    for (int d = 0; d < 4; ++d)
        if ((used >> (8 * d)) & 255u) {
            ++nd;
            dg = d;
        }
    const bool lds_ok = nd == 1;
    if (tid == 0) {  // both roles write the same values (they may run on different streams)
        a.o.mode[bh] = lds_ok ? 1 : 0;
        a.o.onebyte[bh] = nd <= 1 ? 1 : 0;
        a.o.shift[bh] = 8 * dg;  // the top used byte (0 without any)
    }
    // dense rows (classified before the prepare) have no bigram-pair work: role 1 skips them
    // (the owner lists drop them; their label order, role 0, stays, e.g. for the decoder)
    const int dmode = a.o.dflag[bh];
    if (role == 1 && pairless_mode(dmode)) return;
    if (!lds_ok) {
        // the global-memory path takes this row: its combined label order here (the LDS
        // pool as the passes' scratch), the bigram orders in sort_kernel roles 1-2
        if (role == 0) {
            int digits[4], k = 0;
            for (int d = 0; d < 4; ++d)
                if ((used >> (8 * d)) & 255u) digits[k++] = d;
            label_order_global(a, bh, nd, digits, reinterpret_cast<int (*)[RADIX]>(pool),
                               reinterpret_cast<int*>(pool) + SORT_WAVES * RADIX);
        }
        return;
    }
    const int shift = 8 * dg;
    for (int p = tid; p < n; p += SORT_THREADS) {
        s_dig[2 * p] = (uint8_t)(((uint32_t)lk[p] >> shift) & 255u);
        s_dig[2 * p + 1] = (uint8_t)(((uint32_t)lq[p] >> shift) & 255u);
    }
    __syncthreads();
    // ---- combined label order
    lds_pass(
        n2, [&](int x) { return (int)s_dig[x]; },
        [&](int x, int dst) { s_ord[pad(dst)] = (uint16_t)x; },
        role == 0 ? a.o.ctab + (long)bh * (RADIX + 1) : nullptr, wcnt, scan, s_mask);
    if (role == 0) {
        int32_t* corder = a.o.corder + 2 * off;
        int32_t* clab = a.o.clab + 2 * off;
        for (int c = tid; c < n2; c += SORT_THREADS) {
            const int e = s_ord[pad(c)];
            corder[c] = e;
            clab[c] = (int)((uint32_t)s_dig[e] << shift);
        }
        return;
    }
    // ---- combined bigram order: the label order, stably by the predecessor's label (each
    // wave's segment of the label order moves to registers first)
    {
        const int lane = tid & 63, wave = tid >> 6;
        const int seg = ((n2 + SORT_WAVES - 1) / SORT_WAVES + 63) / 64 * 64;
        const int beg = wave * seg, end = beg + seg < n2 ? beg + seg : n2;
        uint32_t vd[32];
#pragma unroll
        for (int g = 0; g < 32; ++g) {
            const int x = beg + 64 * g + lane;
            uint32_t w = (uint32_t)RADIX << 16;
            if (x < end) {
                const int e = s_ord[pad(x)];
                w = (uint32_t)e | ((uint32_t)(e >= 2 ? s_dig[e - 2] : 0) << 16);
            }
            vd[g] = w;
        }
        reg_pass(n2, vd, [&](int e, int dst) { s_ord[pad(dst)] = (uint16_t)e; }, wcnt, scan, s_mask);
    }

    // ---- plan.  Each thread owns PREP_E consecutive entries c of the bigram order; its
    // group-head flags are one register word (bit k: entry c0 + k starts a bigram group).
    const int c0 = tid * PREP_E;
    const int c1 = c0 + PREP_E < n2 ? c0 + PREP_E : n2;
    uint32_t heads = 0;
    {
        auto big_of = [&](int e) {
            return ((e >= 2 ? (int)s_dig[e - 2] : 0) << 8) | (int)s_dig[e];
        };
        int prev = c0 > 0 && c0 <= n2 ? big_of(s_ord[pad(c0 - 1)]) : -1;
#pragma unroll 8
        for (int c = c0; c < c1; ++c) {
            const int b = big_of(s_ord[pad(c)]);
            if (b != prev) heads |= 1u << (c - c0);
            prev = b;
        }
    }
    auto is_head = [&](int c) { return (heads >> (c - c0)) & 1u; };
    // per-thread aggregates: keys, queries (p >= 1); segmented key count after the last head;
    // queries before the first head
    Cnt4 loc{0, 0, 0, 0};
    Seg segk{0, 0}, segq{0, 0};
    for (int c = c0; c < c1; ++c) {
        const int e = s_ord[pad(c)];
        const bool isk = e >= 2 && !(e & 1), isq = e >= 2 && (e & 1);
        if (is_head(c)) {
            segk.f = 1;
            segk.v = 0;
            segq.f = 1;
        }
        segk.v += isk;
        if (!segq.f) segq.v += isq;
        loc.x += isk;
        loc.y += isq;
    }
    auto sh4 = [](Cnt4 v, int l) {
        return Cnt4{__shfl(v.x, l), __shfl(v.y, l), __shfl(v.z, l), __shfl(v.w, l)};
    };
    auto add4 = [](Cnt4 p, Cnt4 q) { return Cnt4{p.x + q.x, p.y + q.y, p.z + q.z, p.w + q.w}; };
    auto shs = [](Seg v, int l) { return Seg{__shfl(v.f, l), __shfl(v.v, l)}; };
    auto segop = [](Seg p, Seg q) { return Seg{p.f | q.f, q.f ? q.v : p.v + q.v}; };
    Cnt4 tot;
    Seg dummy;
    const Cnt4 rk = block_exscan(loc, add4, Cnt4{0, 0, 0, 0}, sh4, s_c4, false, &tot);
    const Seg ck = block_exscan(segk, segop, Seg{0, 0}, shs, s_seg, false, &dummy);
    const Seg cq = block_exscan(segq, segop, Seg{0, 0}, shs, s_seg, true, &dummy);
    // partner counts into s_cnt: keys (queries after them in the group, backward), query
    // rows (keys before them in the group, forward); per-thread class counts
    {
        int qa = cq.v;
        for (int c = c1 - 1; c >= c0; --c) {
            const int e = s_ord[pad(c)];
            const bool isk = e >= 2 && !(e & 1), isq = e >= 2 && (e & 1);
            s_cnt[pad(c)] = isk ? (uint16_t)qa : (uint16_t)0;
            qa += isq;
            if (is_head(c)) qa = 0;
        }
    }
    Cnt4 cl{0, 0, 0, 0}, cl2{0, 0, 0, 0};  // classes of query rows, of keys
    auto add_class = [](Cnt4& cc, int cnt) {
        const int cls = cnt <= OWNER_SMALL ? 0 : cnt <= OWNER_MEDIUM ? 1 : 2;
        cc.x += cls == 0;
        cc.y += cls == 1;
        cc.z += cls == 2;
    };
    {
        int sk = ck.v;
        for (int c = c0; c < c1; ++c) {
            const int e = s_ord[pad(c)];
            const bool isk = e >= 2 && !(e & 1), isq = e >= 2 && (e & 1);
            if (is_head(c)) sk = 0;
            if (isq) {
                s_cnt[pad(c)] = (uint16_t)sk;
                if (sk > 0) add_class(cl, sk);
            } else if (isk) {
                const int cnt = s_cnt[pad(c)];
                if (cnt > 0) add_class(cl2, cnt);
            }
            sk += isk;
        }
    }
    Cnt4 t0, t1;
    Cnt4 r0 = block_exscan(cl, add4, Cnt4{0, 0, 0, 0}, sh4, s_c4, false, &t0);
    Cnt4 r1 = block_exscan(cl2, add4, Cnt4{0, 0, 0, 0}, sh4, s_c4, false, &t1);
    // owner records into the row's stage lists
    {
        int kr = rk.x, qr = rk.y, sk = ck.v;
        for (int c = c0; c < c1; ++c) {
            const int e = s_ord[pad(c)];
            const bool isk = e >= 2 && !(e & 1), isq = e >= 2 && (e & 1);
            if (is_head(c)) sk = 0;
            const int cnt = s_cnt[pad(c)];
            if ((isk || isq) && cnt > 0) {
                const int lo = isq ? kr - sk : qr;
                const int side = isq ? 0 : 1;  // 0: query rows, 1: keys
                const int cls = cnt <= OWNER_SMALL ? 0 : cnt <= OWNER_MEDIUM ? 1 : 2;
                int rank;
                if (side == 0) rank = cls == 0 ? r0.x++ : cls == 1 ? r0.y++ : r0.z++;
                else rank = cls == 0 ? r1.x++ : cls == 1 ? r1.y++ : r1.z++;
                const int4 rec = make_int4(bh, e >> 1, lo, cnt);
                if (cls == 1) a.o.stage[side][1][off + rank] = rec;
                else a.o.stage[side][0][off + (cls == 0 ? rank : n - 1 - rank)] = rec;
            }
            kr += isk;
            qr += isq;
            sk += isk;
        }
    }
    if (tid < 3) {
        a.o.bhcount[0][(long)bh * 4 + tid] = tid == 0 ? t0.x : tid == 1 ? t0.y : t0.z;
        a.o.bhcount[1][(long)bh * 4 + tid] = tid == 0 ? t1.x : tid == 1 ? t1.y : t1.z;
    }
    // per-side bigram position lists, written coalesced: wave-strided groups of 64 entries
    // (two threads' ranges) take their ranks from the threads' prefix counts
    int* s_rk = &wcnt[0][0];  // [SORT_THREADS][2]
    s_rk[2 * tid] = rk.x;
    s_rk[2 * tid + 1] = rk.y;
    __syncthreads();
    {
        const int lane = tid & 63, wave = tid >> 6;
        const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
        int32_t* bq = a.o.bpos[0] + off;
        int32_t* bk = a.o.bpos[1] + off;
        for (int x0 = wave * 64; x0 < n2; x0 += 64 * SORT_WAVES) {
            const int c = x0 + lane;
            const int e = c < n2 ? s_ord[pad(c)] : 0;
            const bool isk = e >= 2 && !(e & 1), isq = e >= 2 && (e & 1);
            const unsigned long long km = __ballot(isk), qm = __ballot(isq);
            const int tb = x0 / PREP_E;
            if (isk) bk[s_rk[2 * tb] + __popcll(km & below)] = e >> 1;
            if (isq) bq[s_rk[2 * tb + 1] + __popcll(qm & below)] = e >> 1;
        }
    }
    // pair counts per query row: zeros here, the owner-list kernel writes the rows with pairs
    for (int p = tid; p < n; p += SORT_THREADS) a.pnb[off + p] = 0;
}

hipError_t launch_prepare_lds(const SortArgs& a, int role0, int roles, hipStream_t s) {
    SortArgs b = a;
    b.role_base = role0;
    hipLaunchKernelGGL(prepare_lds_kernel, dim3((unsigned)a.BH, (unsigned)roles),
                       dim3(SORT_THREADS), 0, s, b);
    return hipGetLastError();
}

hipError_t launch_sort(const SortArgs& a, int role0, int roles, hipStream_t s) {
    SortArgs b = a;
    b.role_base = role0;
    hipLaunchKernelGGL(sort_kernel, dim3((unsigned)a.BH, (unsigned)roles), dim3(SORT_THREADS), 0,
                       s, b);
    return hipGetLastError();
}

hipError_t launch_sort_labels(const SortArgs& a, hipStream_t s) { return launch_msort_labels(a, s); }

// Work buckets of the label scans for rows whose labels differ in more than one byte: the top
// sorted digit can then hold a handful of values (labels 0..511: two), which left one scan
// wave walking hundreds of label groups in series.  Here the 2N entries of the combined order
// are cut into 256 ranges of about 2N/256 entries, each boundary moved forward to the next
// label change (upper bound of the label before it), so every label group stays whole.
// One workgroup per row, thread b computes boundary b.
__global__ __launch_bounds__(256) void ctab_balance_kernel(const int32_t* __restrict__ clab_all,
                                                           const int32_t* __restrict__ onebyte,
                                                           int32_t* __restrict__ ctab_all,
                                                           int n) {
    const long bh = blockIdx.x;
    if (onebyte[bh]) return;
    const int tid = (int)threadIdx.x, n2 = 2 * n;
    const int32_t* clab = clab_all + bh * n2;
    int32_t* ctab = ctab_all + bh * (RADIX + 1);
    int x = 0;
    if (tid > 0) {
        const int t = (int)((long)tid * n2 / RADIX);
        // first index in [t, n2) whose (unsigned) label exceeds the one before t
        const uint32_t prev = (uint32_t)clab[t - 1];
        int lo = t, hi = n2;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if ((uint32_t)clab[mid] <= prev) lo = mid + 1; else hi = mid;
        }
        x = lo;
    }
    ctab[tid] = x;
    if (tid == 0) ctab[RADIX] = n2;
}

hipError_t launch_ctab_balance(const SortArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(ctab_balance_kernel, dim3((unsigned)a.BH), dim3(RADIX), 0, s, a.o.clab,
                       a.o.onebyte, a.o.ctab, a.n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Level lists, sequentially (one 1024-thread workgroup per dense row, after the
// classification; rows of N <= LEVEL_MAX_N whose labels are all below 256 but not all below
// 16 -- those go to level_lvl_kernel -- fixed-length calls without resets).
// Level l's list is the previous level's kept list without its entries at p = l - 2, stably
// sorted by label[p - l + 1] (entry e's digit at level l is s_lab[e - 2(l - 1)], the labels
// staged in LDS as bytes).  A group (equal digit and equal previous group) is kept when one
// of its queries has a key before it.  Per level: the stable partition by digit
// (lds_pass), one block scan for every entry's group
// start, keys before it in the group and the last of them, the keep flags, one block scan for
// the kept entries (written out with their key counts) and the next level's input (kept,
// p >= l).  The row becomes mode 3 when a level keeps nothing within
// LEVEL_MAX levels and LEVEL_BUDGET * N kept entries; otherwise it stays a mode-1 (tile)
// row.  The oracle's levels_build computes the same lists.
namespace {
struct LvAgg {  // segmented aggregate of a run of list entries
    int f, cnt, lk, gs;  // a group start inside; keys / last key position after the last
                         // start; index of the last start (-1: none)
};
__device__ __forceinline__ LvAgg lv_op(LvAgg a, LvAgg b) {
    return LvAgg{a.f | b.f, b.f ? b.cnt : a.cnt + b.cnt, b.f || b.lk >= 0 ? b.lk : a.lk,
                 b.gs >= 0 ? b.gs : a.gs};
}


// A stable counting pass as lds_pass, with the ranks inside a 64-element group from ballot
// matching of the 9-bit digit (no rank-mask scratch, so two level workgroups fit a CU).
template <typename Dig, typename Emit>
__device__ void lv_pass(int m, Dig digit, Emit emit, int (*wcnt)[RADIX], int* scan) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int seg = ((m + SORT_WAVES - 1) / SORT_WAVES + 63) / 64 * 64;
    const int beg = wave * seg;
    const int end = beg + seg < m ? beg + seg : m;
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int e = tid; e < SORT_WAVES * RADIX; e += SORT_THREADS) (&wcnt[0][0])[e] = 0;
    __syncthreads();
    for (int x0 = beg; x0 < end; x0 += 64) {
        const int x = x0 + lane;
        const int dig = x < end ? digit(x) : RADIX;
        const unsigned long long eq = match_digit(dig);
        if (dig < RADIX && !(eq & below)) wcnt[wave][dig] += __popcll(eq);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    if (tid < RADIX) {
        int tot = 0;
        for (int w = 0; w < SORT_WAVES; ++w) tot += wcnt[w][tid];
        scan[tid] = tot;
    }
    __syncthreads();
    if (tid < 64) {
        const int v0 = scan[4 * tid], v1 = scan[4 * tid + 1], v2 = scan[4 * tid + 2],
                  v3 = scan[4 * tid + 3];
        const int sum = v0 + v1 + v2 + v3;
        int inc = sum;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(inc, off);
            if (lane >= off) inc += t;
        }
        int ex = inc - sum;
        scan[4 * tid] = ex;
        ex += v0;
        scan[4 * tid + 1] = ex;
        ex += v1;
        scan[4 * tid + 2] = ex;
        ex += v2;
        scan[4 * tid + 3] = ex;
    }
    __syncthreads();
    if (tid < RADIX) {
        int run = scan[tid];
        for (int w = 0; w < SORT_WAVES; ++w) {
            const int c = wcnt[w][tid];
            wcnt[w][tid] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int x0 = beg; x0 < end; x0 += 64) {
        const int x = x0 + lane;
        const int dig = x < end ? digit(x) : RADIX;
        const unsigned long long eq = match_digit(dig);
        const int rank = __popcll(eq & below);
        const int dst = dig < RADIX ? wcnt[wave][dig] + rank : 0;
        __builtin_amdgcn_wave_barrier();
        if (dig < RADIX && rank == 0) wcnt[wave][dig] += __popcll(eq);
        __builtin_amdgcn_wave_barrier();
        if (x < end) emit(x, dst);
    }
    __syncthreads();
}
}  // namespace

__global__ __launch_bounds__(SORT_THREADS) void level_prep_kernel(PathArgs a) {
    constexpr int M2 = 2 * LEVEL_MAX_N;
    __shared__ uint16_t s_e[2][M2];
    __shared__ uint16_t s_g[2][M2];
    __shared__ uint8_t s_lab[M2];
    __shared__ uint8_t s_keep[M2];
    __shared__ int wcnt[SORT_WAVES][RADIX];
    __shared__ int scan[RADIX];
    __shared__ unsigned long long lmask[SORT_WAVES][RADIX];
    __shared__ LvAgg s_agg[SORT_WAVES];
    __shared__ Cnt4 s_c4[SORT_WAVES];
    __shared__ uint32_t s_or;
    // per position: longest match, kept levels of the query / the key, the longest match's
    // last key (0xFFFF: none); written out once at the end
    __shared__ uint8_t s_lq[LEVEL_MAX_N], s_kq[LEVEL_MAX_N], s_kk[LEVEL_MAX_N];
    __shared__ uint16_t s_jarg[LEVEL_MAX_N];
    // nv: the positions the lists take (a prefill's padding after them never pairs with
    // them: its keys come after every real query)
    const int bh = blockIdx.x, tid = threadIdx.x, n = a.n;
    const int nv = a.cls_n > 0 && a.cls_n < n ? a.cls_n : n, n2 = 2 * nv;
    if (a.o.dflag[bh] != 1) return;
    const long so = (long)bh * n;
    const int32_t* q = a.iq + so;
    const int32_t* k = a.ik + so;
    if (tid == 0) s_or = 0;
    __syncthreads();
    uint32_t orv = 0;
    for (int p = tid; p < nv; p += SORT_THREADS) {
        const uint32_t lq = (uint32_t)q[p], lk = (uint32_t)k[p];
        orv |= lq | lk;
        s_lab[2 * p] = (uint8_t)lk;
        s_lab[2 * p + 1] = (uint8_t)lq;
        s_e[0][2 * p] = (uint16_t)(2 * p);
        s_e[0][2 * p + 1] = (uint16_t)(2 * p + 1);
        s_g[0][2 * p] = 0;
        s_g[0][2 * p + 1] = 0;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) orv |= (uint32_t)__shfl_xor((int)orv, o);
    if ((tid & 63) == 0 && orv) atomicOr(&s_or, orv);
    __syncthreads();
    const uint32_t used = s_or;
    // labels of more than one byte: not a level row; below 16: level_lvl_kernel's rows
    if (used >= 256u || used < 16u) return;
    int32_t* ent = a.o.lvent + (long)bh * LEVEL_MAX * 2 * n;
    int32_t* meta = a.o.lvmeta + (long)bh * LEVEL_META;
    for (int p = tid; p < n; p += SORT_THREADS) {
        s_lq[p] = 0;
        s_kq[p] = 0;
        s_kk[p] = 0;
        s_jarg[p] = 0xFFFF;
    }
    auto sh4 = [](Cnt4 v, int l) {
        return Cnt4{__shfl(v.x, l), __shfl(v.y, l), __shfl(v.z, l), __shfl(v.w, l)};
    };
    auto add4 = [](Cnt4 p, Cnt4 r) { return Cnt4{p.x + r.x, p.y + r.y, p.z + r.z, p.w + r.w}; };
    auto sha = [](LvAgg v, int l) {
        return LvAgg{__shfl(v.f, l), __shfl(v.cnt, l), __shfl(v.lk, l), __shfl(v.gs, l)};
    };
    int cur = 0, m = n2, total = 0, segs = 0, nlev = -1;
    if (tid == 0) {
        meta[1] = 0;                    // off[0]
        meta[LEVEL_MAX + 2] = 0;        // segbase[0]
    }
    for (int l = 1; l <= LEVEL_MAX + 1; ++l) {
        const int oth = cur ^ 1;
        const int sh = 2 * (l - 1);
        for (int c = tid; c < m; c += SORT_THREADS) s_keep[c] = 0;
        // ---- stable partition by label[p - l + 1]: cur -> oth
        auto dig = [&](int x) { return (int)s_lab[s_e[cur][x] - sh]; };
        auto emit = [&](int x, int dst) {
            s_e[oth][dst] = s_e[cur][x];
            s_g[oth][dst] = s_g[cur][x];
        };
        lds_pass(m, dig, emit, nullptr, wcnt, scan, lmask);
        // ---- groups: start, keys before, last key; keep flags
        const int ept = (m + SORT_THREADS - 1) / SORT_THREADS;
        const int c0 = tid * ept, c1 = c0 + ept < m ? c0 + ept : m;
        auto is_start = [&](int c) {
            if (c == 0) return true;
            const int e = s_e[oth][c], f = s_e[oth][c - 1];
            return s_lab[e - sh] != s_lab[f - sh] || s_g[oth][c] != s_g[oth][c - 1];
        };
        LvAgg loc{0, 0, -1, -1};
        uint32_t starts = 0;  // bit c - c0: entry c starts a group
        for (int c = c0; c < c1; ++c) {
            const int e = s_e[oth][c];
            const bool st = is_start(c);
            starts |= (st ? 1u : 0u) << (c - c0);
            const LvAgg one{st ? 1 : 0, (e & 1) ? 0 : 1, (e & 1) ? -1 : (e >> 1), st ? c : -1};
            loc = lv_op(loc, one);
        }
        LvAgg dummy;
        const LvAgg pre = block_exscan(loc, lv_op, LvAgg{0, 0, -1, -1}, sha, s_agg, false, &dummy);
        {
            LvAgg run = pre;
            for (int c = c0; c < c1; ++c) {
                const int e = s_e[oth][c];
                if ((starts >> (c - c0)) & 1u) run = LvAgg{1, 0, -1, c};
                if ((e & 1) && run.cnt > 0) s_keep[run.gs] = 1;
                if (!(e & 1)) ++run.cnt;
            }
        }
        __syncthreads();
        // ---- kept entries (x) and the next level's input (y: kept, p >= l)
        Cnt4 kn{0, 0, 0, 0};
        {
            int gs = pre.gs;
            for (int c = c0; c < c1; ++c) {
                if ((starts >> (c - c0)) & 1u) gs = c;
                const int kp = s_keep[gs];
                kn.x += kp;
                kn.y += kp && (s_e[oth][c] >> 1) >= l;
            }
        }
        Cnt4 kt;
        Cnt4 kb = block_exscan(kn, add4, Cnt4{0, 0, 0, 0}, sh4, s_c4, false, &kt);
        if (kt.x == 0) {
            nlev = l - 1;
            break;
        }
        if (l == LEVEL_MAX + 1 || total + kt.x > LEVEL_BUDGET * nv) break;  // not a level row
        {
            LvAgg run = pre;
            for (int c = c0; c < c1; ++c) {
                const int e = s_e[oth][c];
                const bool st = (starts >> (c - c0)) & 1u;
                if (st) run = LvAgg{1, 0, -1, c};
                if (s_keep[run.gs]) {
                    const int idx = kb.x++;
                    const int p = e >> 1;
                    ent[(long)(l - 1) * 2 * n + idx] =
                        e | ((e & 1) ? run.cnt << LEVEL_EBITS : 0) | (st ? LEVEL_START : 0);
                    if (p >= l) {  // next level's input (its group id: kept index of the start)
                        s_e[cur][kb.y] = (uint16_t)e;
                        s_g[cur][kb.y] = (uint16_t)(idx - (c - run.gs));
                        ++kb.y;
                    }
                    if (e & 1) {
                        s_kq[p] = (uint8_t)l;
                        if (run.cnt > 0) {
                            s_lq[p] = (uint8_t)l;
                            s_jarg[p] = (uint16_t)run.lk;
                        }
                    } else {
                        s_kk[p] = (uint8_t)l;
                    }
                }
                if (!(e & 1)) {
                    run.cnt += 1;
                    run.lk = e >> 1;
                }
            }
        }
        __syncthreads();
        total += kt.x;
        segs += (kt.x + LEVEL_SEG - 1) / LEVEL_SEG;
        if (tid == 0) {
            meta[1 + l] = total;
            meta[LEVEL_MAX + 2 + l] = segs;
        }
        m = kt.y;
    }
    if (nlev <= 0) return;  // not a level row (uniform)
    int4* lq = a.o.lvq + so;
    for (int p = tid; p < n; p += SORT_THREADS)
        lq[p] = make_int4(s_lq[p], s_jarg[p] == 0xFFFF ? -1 : (int)s_jarg[p], s_kq[p], s_kk[p]);
    if (tid == 0) {
        meta[0] = nlev;
        a.o.dflag[bh] = 3;
    }
}

// Level lists, one level per workgroup (grid (B*H, LEVEL_MAX + 1)), for rows whose labels
// are all below 16.  The level-l list is the same as the sequential construction's: the
// entries at p >= l - 1 ordered by their l-gram read oldest label first, then by e, without
// the groups that hold no valid pair (a group's sub-groups hold none either, so the lists do
// not depend on the previous level).  With b-bit symbols (b = 1, 2 or 4), byte k of the
// l-gram key is the packed history s_h8[e - 2 S k] of S = 8 / b labels (the oldest of them
// in its top bits, the last byte masked to the l-gram); LSD passes over the key bytes
// (lds_pass) give the order.  The per-position flags and last keys go to lvlf / lvlk, the
// kept count to lvlc[l]; level_finalize_kernel then takes the row to mode 3 or leaves it.
__global__ __launch_bounds__(SORT_THREADS) void level_lvl_kernel(PathArgs a, int l0) {
    constexpr int M2 = 2 * LEVEL_MAX_N;
    // (under 80 KiB, so that two workgroups share a CU: the labels' bytes and later the
    // per-position flags share one region, the keep flags use the idle order buffer)
    __shared__ uint16_t s_e[2][M2];
    __shared__ uint32_t s_u[LEVEL_MAX_N];   // s_lab (bytes), then s_fl
    __shared__ uint8_t s_h8[M2];
    __shared__ int wcnt[SORT_WAVES][RADIX];
    __shared__ int scan[RADIX];
    __shared__ LvAgg s_agg[SORT_WAVES];
    __shared__ Cnt4 s_c4[SORT_WAVES];
    __shared__ uint32_t s_or;
    uint8_t* s_lab = reinterpret_cast<uint8_t*>(s_u);
    uint32_t* s_fl = s_u;
    const int bh = blockIdx.x, l = (int)blockIdx.y + l0, tid = threadIdx.x, n = a.n;
    const int nv = a.cls_n > 0 && a.cls_n < n ? a.cls_n : n;
    if (a.o.dflag[bh] != 1) return;
    // a later launch's levels: nothing to do once an earlier level kept nothing
    if (l0 > 1 && a.o.lvlc[(long)bh * (LEVEL_MAX + 2) + l0 - 1] == 0) {
        if (tid == 0) a.o.lvlc[(long)bh * (LEVEL_MAX + 2) + l] = 0;
        return;
    }
    const long so = (long)bh * n;
    const int32_t* q = a.iq + so;
    const int32_t* k = a.ik + so;
    if (tid == 0) s_or = 0;
    __syncthreads();
    uint32_t orv = 0;
    for (int p = tid; p < nv; p += SORT_THREADS) {
        const uint32_t lq = (uint32_t)q[p], lk = (uint32_t)k[p];
        orv |= lq | lk;
        s_lab[2 * p] = (uint8_t)lk;
        s_lab[2 * p + 1] = (uint8_t)lq;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) orv |= (uint32_t)__shfl_xor((int)orv, o);
    if ((tid & 63) == 0 && orv) atomicOr(&s_or, orv);
    __syncthreads();
    const uint32_t used = s_or;
    if (used >= 16u) return;  // the sequential construction's rows
    const int b = used < 2u ? 1 : used < 4u ? 2 : 4, S = 8 / b;
    int32_t* cnts = a.o.lvlc + (long)bh * (LEVEL_MAX + 2);
    uint8_t* lf = a.o.lvlf + ((long)bh * (LEVEL_MAX + 1) + (l - 1)) * n;
    const int e0 = 2 * (l - 1), m = 2 * nv - e0;
    if (m <= 0) {
        for (int p = tid; p < n; p += SORT_THREADS) lf[p] = 0;
        if (tid == 0) cnts[l] = 0;
        return;
    }
    for (int e = tid; e < 2 * nv; e += SORT_THREADS) {
        const int qp = e >> 1, side = e & 1;
        uint32_t h = 0;
        for (int u = 0; u < S && qp - u >= 0; ++u) h |= (uint32_t)s_lab[2 * (qp - u) + side] << (b * u);
        s_h8[e] = (uint8_t)h;
    }
    for (int x = tid; x < m; x += SORT_THREADS) s_e[0][x] = (uint16_t)(e0 + x);
    __syncthreads();
    for (int p = tid; p < nv; p += SORT_THREADS) s_fl[p] = 0u;  // (the labels are in s_h8 now)
    const int nbytes = (l + S - 1) / S;
    const int lastmask = (l % S) ? (1 << (b * (l - S * (nbytes - 1)))) - 1 : 0xFF;
    auto kbyte = [&](int e, int kk) {
        const int v = s_h8[e - 2 * S * kk];
        return kk == nbytes - 1 ? (v & lastmask) : v;
    };
    int cur = 0;
    for (int kk = 0; kk < nbytes; ++kk) {
        const int nx = cur ^ 1;
        lv_pass(
            m, [&](int x) { return kbyte(s_e[cur][x], kk); },
            [&](int x, int dst) { s_e[nx][dst] = s_e[cur][x]; }, wcnt, scan);
        cur = nx;
    }
    uint8_t* s_keep = reinterpret_cast<uint8_t*>(s_e[cur ^ 1]);
    // ---- groups, keep flags, compaction (as the sequential construction's level step)
    const int ept = (m + SORT_THREADS - 1) / SORT_THREADS;
    const int c0 = tid * ept, c1 = c0 + ept < m ? c0 + ept : m;
    auto is_start = [&](int c) {
        if (c == 0) return true;
        const int e = s_e[cur][c], f = s_e[cur][c - 1];
        for (int kk = 0; kk < nbytes; ++kk)
            if (kbyte(e, kk) != kbyte(f, kk)) return true;
        return false;
    };
    for (int c = tid; c < m; c += SORT_THREADS) s_keep[c] = 0;
    LvAgg loc{0, 0, -1, -1};
    uint32_t starts = 0;
    for (int c = c0; c < c1; ++c) {
        const int e = s_e[cur][c];
        const bool st = is_start(c);
        starts |= (st ? 1u : 0u) << (c - c0);
        const LvAgg one{st ? 1 : 0, (e & 1) ? 0 : 1, (e & 1) ? -1 : (e >> 1), st ? c : -1};
        loc = lv_op(loc, one);
    }
    auto sha = [](LvAgg v, int ln) {
        return LvAgg{__shfl(v.f, ln), __shfl(v.cnt, ln), __shfl(v.lk, ln), __shfl(v.gs, ln)};
    };
    LvAgg dummy;
    const LvAgg pre = block_exscan(loc, lv_op, LvAgg{0, 0, -1, -1}, sha, s_agg, false, &dummy);
    {
        LvAgg run = pre;
        for (int c = c0; c < c1; ++c) {
            const int e = s_e[cur][c];
            if ((starts >> (c - c0)) & 1u) run = LvAgg{1, 0, -1, c};
            if ((e & 1) && run.cnt > 0) s_keep[run.gs] = 1;
            if (!(e & 1)) ++run.cnt;
        }
    }
    __syncthreads();
    Cnt4 kn{0, 0, 0, 0};
    {
        int gs = pre.gs;
        for (int c = c0; c < c1; ++c) {
            if ((starts >> (c - c0)) & 1u) gs = c;
            kn.x += s_keep[gs];
        }
    }
    auto sh4 = [](Cnt4 v, int ln) {
        return Cnt4{__shfl(v.x, ln), __shfl(v.y, ln), __shfl(v.z, ln), __shfl(v.w, ln)};
    };
    auto add4 = [](Cnt4 x, Cnt4 y) { return Cnt4{x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w}; };
    Cnt4 kt;
    Cnt4 kb = block_exscan(kn, add4, Cnt4{0, 0, 0, 0}, sh4, s_c4, false, &kt);
    if (l <= LEVEL_MAX && kt.x > 0) {
        int32_t* ent = a.o.lvent + (long)bh * LEVEL_MAX * 2 * n + (long)(l - 1) * 2 * n;
        uint16_t* lk = a.o.lvlk + ((long)bh * LEVEL_MAX + (l - 1)) * n;
        LvAgg run = pre;
        for (int c = c0; c < c1; ++c) {
            const int e = s_e[cur][c];
            const bool st = (starts >> (c - c0)) & 1u;
            if (st) run = LvAgg{1, 0, -1, c};
            if (s_keep[run.gs]) {
                const int idx = kb.x++;
                const int p = e >> 1;
                ent[idx] = e | ((e & 1) ? run.cnt << LEVEL_EBITS : 0) | (st ? LEVEL_START : 0);
                if (e & 1) {
                    atomicOr(&s_fl[p], run.cnt > 0 ? 3u : 1u);
                    if (run.cnt > 0) lk[p] = (uint16_t)run.lk;
                } else {
                    atomicOr(&s_fl[p], 4u);
                }
            }
            if (!(e & 1)) {
                run.cnt += 1;
                run.lk = e >> 1;
            }
        }
    }
    __syncthreads();
    for (int p = tid; p < n; p += SORT_THREADS) lf[p] = p < nv ? (uint8_t)s_fl[p] : 0;
    if (tid == 0) cnts[l] = kt.x;
}

// Mode 3 for the rows level_lvl_kernel built whose levels end within LEVEL_MAX and the
// budget; the level offsets, segment bases and per-position summaries.  Grid (B*H, slices of
// 256 positions): every workgroup of a row decides the same way from the row's level
// counts; slice 0 writes the row's offsets and mode, slice y the summaries of its positions.
// A slice may start after slice 0 has set mode 3, so mode 3 counts as "dense" here (no other
// kernel sets it before this one).
__global__ __launch_bounds__(256) void level_finalize_kernel(PathArgs a) {
    __shared__ uint32_t s_or;
    __shared__ int s_nlev;
    const int bh = blockIdx.x, tid = threadIdx.x, n = a.n, y = blockIdx.y;
    const int nv = a.cls_n > 0 && a.cls_n < n ? a.cls_n : n;
    const int f = a.o.dflag[bh];
    if (f != 1 && f != 3) return;
    const long so = (long)bh * n;
    if (tid == 0) s_or = 0;
    __syncthreads();
    uint32_t orv = 0;
    for (int p = tid; p < nv; p += 256) orv |= (uint32_t)a.iq[so + p] | (uint32_t)a.ik[so + p];
    if (orv) atomicOr(&s_or, orv);
    __syncthreads();
    if (s_or >= 16u) return;
    const int32_t* cnts = a.o.lvlc + (long)bh * (LEVEL_MAX + 2);
    int32_t* meta = a.o.lvmeta + (long)bh * LEVEL_META;
    if (tid < 64) {  // lane l - 1 holds level l's count
        const int c = tid < LEVEL_MAX + 1 ? cnts[tid + 1] : 0;
        const unsigned long long z = __ballot(tid < LEVEL_MAX + 1 && c == 0);
        int nlev = z ? __builtin_ctzll(z) : -1, total = 0;
        if (nlev > 0) {
            int segs = 0;
            if (y == 0 && tid == 0) {
                meta[1] = 0;
                meta[LEVEL_MAX + 2] = 0;
            }
            for (int l = 1; l <= nlev; ++l) {
                const int cl = __shfl(c, l - 1);
                total += cl;
                segs += (cl + LEVEL_SEG - 1) / LEVEL_SEG;
                if (y == 0 && tid == 0) {
                    meta[1 + l] = total;
                    meta[LEVEL_MAX + 2 + l] = segs;
                }
            }
            if (total > LEVEL_BUDGET * nv) nlev = -1;
        }
        if (tid == 0) s_nlev = nlev;
    }
    __syncthreads();
    const int nlev = s_nlev;
    if (nlev <= 0) return;
    const uint8_t* lf = a.o.lvlf + (long)bh * (LEVEL_MAX + 1) * n;
    const uint16_t* lk = a.o.lvlk + (long)bh * LEVEL_MAX * n;
    for (int p = y * 256 + tid; p < n && p < (y + 1) * 256; p += 256) {
        int kq = 0, lq = 0, kk = 0;
        for (int l0 = 1; l0 <= nlev; l0 += 8) {  // eight levels' loads in flight
            int f[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) f[u] = l0 + u <= nlev ? lf[(long)(l0 + u - 1) * n + p] : 0;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (f[u] & 1) kq = l0 + u;
                if (f[u] & 2) lq = l0 + u;
                if (f[u] & 4) kk = l0 + u;
            }
        }
        a.o.lvq[so + p] = make_int4(lq, lq > 0 ? (int)lk[(long)(lq - 1) * n + p] : -1, kq, kk);
    }
    if (y == 0 && tid == 0) {
        meta[0] = nlev;
        a.o.dflag[bh] = 3;
    }
}

hipError_t launch_level_prep(const PathArgs& a, hipStream_t s) {
    if (!a.o.lvent || a.dstart || a.wlo || a.n > LEVEL_MAX_N) return hipSuccess;
    const unsigned BH = (unsigned)(a.B * a.H);
    // levels 1..16, then 17..33 (those exit at once when level 16 kept nothing)
    hipLaunchKernelGGL(level_lvl_kernel, dim3(BH, 16), dim3(SORT_THREADS), 0, s, a, 1);
    hipLaunchKernelGGL(level_lvl_kernel, dim3(BH, LEVEL_MAX + 1 - 16), dim3(SORT_THREADS), 0, s,
                       a, 17);
    hipLaunchKernelGGL(level_finalize_kernel, dim3(BH, (unsigned)((a.n + 255) / 256)),
                       dim3(256), 0, s, a);
    hipLaunchKernelGGL(level_prep_kernel, dim3(BH), dim3(SORT_THREADS), 0, s, a);
    return hipGetLastError();
}

}  // namespace dism
