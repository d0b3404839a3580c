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

// grid (BH, 3)
__global__ __launch_bounds__(SORT_THREADS) void sort_kernel(SortArgs a) {
    __shared__ int wcnt[SORT_WAVES][RADIX];
    __shared__ int scan[RADIX];
    __shared__ uint32_t mask;
    const int bh = blockIdx.x, role = blockIdx.y, n = a.n, tid = threadIdx.x;
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
    if (tid == 0 && role == 0) a.o.shift[bh] = nd ? 8 * digits[nd - 1] : 0;

    if (role == 0) {
        // ---- combined label order of the 2N entries
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

hipError_t launch_sort(const SortArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(sort_kernel, dim3((unsigned)a.BH, 3), dim3(SORT_THREADS), 0, s, a);
    return hipGetLastError();
}

}  // namespace dism
