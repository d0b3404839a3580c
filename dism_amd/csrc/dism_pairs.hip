// dism_pairs.hip -- bigram pairs: the corrections of matches with L >= 2.
//
// A valid pair (j <= i, iq[i] == ik[j]) has L >= 2 exactly when i, j >= 1 and
// iq[i-1] == ik[j-1], i.e. when the (previous label, label) bigrams of i and j are equal.
// Bigram orders (dism_sort.hip) make each bigram group one contiguous, position-ascending
// range, so an owner (a query row, or a key) finds its partners with binary searches and
// visits only them.  Each pair's length comes from the suffix walk (bounded by the composed
// carry boundary when one is given).
//
// Mapping (MI355X): the plan kernel sorts the owners that have partners into three classes
// by partner count; a wave takes 64/G owners of one class with G lanes per owner ("slot"):
//   small  (cnt <= 4):  G = 4,  16 owners per wave;
//   medium (cnt <= 16): G = 16, 4 owners per wave;
//   large:              G = 64, 1 owner per wave.
// (With 256 symbols and long rows, most owners have one partner and few more than four.)
// An owner's partners are consumed in rounds of G (one round for all but the large class
// beyond 64 partners), so a wave's dependent-load chain does not grow with the longest
// partner list among many owners.  Per round:
//   phase A  lane = (slot, sub): the round's pair c0 + sub -- walk, exp2, dot products (the
//            owner's own DV-row staged in LDS) -- with the per-pair coefficients put in LDS;
//   phase B  lane = (slot, column group): each slot folds its round's pairs into its own
//            running sums in ascending partner order (partner value rows are loaded straight
//            from HBM, a few pairs at a time).
// The kernels are persistent: a fixed grid of waves strides over the items of all three
// classes.  The longest-match statistics are order-free maxima (LDS atomics).
// fp32 sequences (repeated by the CPU model), per owner over its pairs in ascending partner
// position:
//   forward rows: m = max(0, LUT[1], LUT[L]); p1 = exp2(LUT[1]-m); p = exp2(LUT[L]-m);
//     dp = dp + p; s = chain(sq.sk); corr[d] = fma((p - p1)*s, v_j[d], corr[d]);
//     den = (exp2(-m) + (float)(cnt - nb)*p1) + dp; out[d] = fma(p1, y[d], corr[d]) * (1/den)
//   backward rows (l2 = lse2_i, cc = G[i+1]): P1 = exp2(LUT[1]-l2); q1 = P1*(G[1]-cc);
//     p = exp2(LUT[L]-l2); dp = p-P1; s = chain(sq.sk); e = tree(dO_i.v_j) (below);
//     g = G[L]-cc; a = p*g - q1;
//     cdq[r] = fma(dp*e, sk[r], cdq[r]); cu = fma(dp*s, e, cu); cvv += a;
//     cw = fma(a, s*e, cw); cz += dp
//   backward keys: p = exp2(LUT[L]-l2_i); dp = p - exp2(LUT[1]-l2_i);
//     cdk[r] = fma(dp*e, sq_i[r], cdk[r]); cdv[d] = fma(dp*s, dO_i[d], cdv[d]);
//     dsk[r] += cdk[r]; dv[d] += cdv[d].
#include "dism_path.h"

DISM_TU_LAYOUT(pairs)

namespace dism {

constexpr int PAIR_SLOTS = 64;        // pairs per wave per round (one per lane)
// Lanes per owner of the small and medium classes: at least the class's partner bound (so
// its owners finish in one round); wider slots where the kernel's per-lane value registers
// (DV / lanes columns, several rows at a time) would not fit otherwise (the key kernel, which
// also keeps its own row and two accumulators per column, and DV = 128).
__host__ __device__ constexpr int lanes_small(int dv, bool keys) {
    return keys || dv >= 128 ? 8 : OWNER_SMALL;
}
__host__ __device__ constexpr int lanes_medium(int dv) { return dv >= 128 ? 32 : OWNER_MEDIUM; }
constexpr int LANES_SMALL_MIN = OWNER_SMALL;  // most small-class slots per wave: 64 / 4
// partner rows per batch of the one-round path and per step of the ordered accumulation:
// about 32 registers of row values per lane
__host__ __device__ constexpr int row_batch(int cpl, int cap) {
    return 32 / cpl < 2 ? 2 : (32 / cpl > cap ? cap : 32 / cpl);
}
constexpr unsigned PAIR_GRID = 2048;  // workgroups of the persistent pair kernels

// Partner range of owner t of side SIDE's bigram order (0: query rows with key partners
// 1 <= j <= i; 1: keys with query partners i >= j): [lo, lo + cnt) of the other side's
// bigram order.
template <int SIDE>
__device__ __forceinline__ void partner_range(const PathArgs& a, int bh, long so, int t, int p,
                                              int& lo_out, int& cnt_out) {
    constexpr int OTHER = 1 - SIDE;
    int lo = 0, hi = 0;
    if (p >= 1) {
        bigram_range(a.o.bplab[OTHER] + so, a.o.blab[OTHER] + so,
                     a.o.btab[OTHER] + (long)bh * 257, a.o.shift[bh],
                     (uint32_t)a.o.bplab[SIDE][so + t], (uint32_t)a.o.blab[SIDE][so + t], lo,
                     hi);
        const int32_t* ob = a.o.bpos[OTHER] + so;
        // packed rows: the diagonal pair (p, p) at a document start p has predecessors in
        // the previous document and is not a bigram pair
        const bool dstart = a.dstart && a.dstart[p] == p;
        if (SIDE == 0) {
            if (lo < hi && ob[lo] == 0) ++lo;  // key 0 has no predecessor
            int l = lo, r = hi;                // keys j <= i
            while (l < r) {
                const int mid = (l + r) >> 1;
                if (ob[mid] <= p) l = mid + 1; else r = mid;
            }
            hi = l;
            if (dstart && hi > lo && ob[hi - 1] == p) --hi;
        } else {
            int l = lo, r = hi;                // queries i >= j
            while (l < r) {
                const int mid = (l + r) >> 1;
                if (ob[mid] < p) l = mid + 1; else r = mid;
            }
            lo = l;
            if (dstart && lo < hi && ob[lo] == p) ++lo;
        }
    }
    lo_out = lo;
    cnt_out = hi - lo;
}

// one step of a suffix walk at offset c: compares the PF label pairs (i - c - u, j - c - u),
// advances c over the matching ones; true when all PF matched (the walk goes on)
template <int PF>
__device__ __forceinline__ bool walk_step(const int32_t* __restrict__ q,
                                          const int32_t* __restrict__ k, int i, int j, int lo,
                                          int& c) {
    int qv[PF], kv[PF];
#pragma unroll
    for (int u = 0; u < PF; ++u) {
        const int iq = i - c - u, jk = j - c - u;
        qv[u] = q[iq > 0 ? iq : 0];
        kv[u] = k[jk > 0 ? jk : 0];
    }
    int run = 0;
#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (run == u && i - c - u >= lo && j - c - u >= 0 && qv[u] == kv[u]) ++run;
    c += run;
    return run == PF;
}

// Match length of a bigram pair (i, j >= 1, q[i-1] == k[j-1] known): match_length's suffix
// walk without its first comparison.
// dlo: the lowest query position the walk may reach (walk_lo: document start, last reset;
// calls with either have no carry boundary).
// wb: the row's 16-bit strip boundaries (rows whose walks the probe found long, mode 2): the
// walk stops at its 64-row strip's first row i0 and adds L[i0 - 1, j - c] from the boundary
// row (unless a reset or document start at or above i0 ends the walk first).
// The listed long runs of a row (sorted by diagonal, then end), or none.
struct RunList {
    const int4* p;
    int n;
};
__device__ __forceinline__ RunList runs_of(const PathArgs& a, int bh) {
    RunList r{nullptr, 0};
    if (a.o.runs && !a.wlo && !a.dstart && !a.bound) {
        const int c = a.o.runcnt[bh];
        if (c <= RUN_CAP) {  // a complete list
            r.p = a.o.runs + (long)bh * RUN_CAP;
            r.n = c;
        }
    }
    return r;
}

// length of the pair (i, j) inside a listed run: the run on diagonal i - j whose end is the
// first at or after i; -1 when there is none covering i
__device__ __forceinline__ int run_length(const RunList& rl, int i, int j) {
    const int d = i - j;
    int lo = 0, hi = rl.n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        const int4 r = rl.p[mid];
        if (r.x < d || (r.x == d && r.y < i)) lo = mid + 1;
        else hi = mid;
    }
    if (lo < rl.n) {
        const int4 r = rl.p[lo];
        if (r.x == d && r.y - r.z < i) return r.z - (r.y - i);
    }
    return -1;
}

__device__ __forceinline__ int pair_length(const int32_t* __restrict__ q,
                                           const int32_t* __restrict__ k, int i, int j,
                                           const int32_t* __restrict__ bound, int strip, int n,
                                           int dlo, const uint16_t* __restrict__ wb = nullptr,
                                           RunList rl = RunList{nullptr, 0}) {
    const int s0 = wb ? (i & ~63) : 0;
    const int lo = bound ? (i / strip) * strip : (s0 > dlo ? s0 : dlo);
    int c = i - 1 >= lo ? 2 : 1;
    // the walk compares a batch of label pairs per step, all loads in flight together
    // (clamped indices; a comparison counts only while both positions are in range): 4 at
    // first, so the usual short match costs one round trip, then 16 per step for long runs;
    // a walk that reaches RUN_MIN labels takes its length from its run's listed end
    if (c == 2 && walk_step<4>(q, k, i, j, lo, c)) {
        bool on = true;
        while (on && c < RUN_MIN) on = walk_step<16>(q, k, i, j, lo, c);
        if (on && rl.n > 0 && !wb) {
            const int L = run_length(rl, i, j);
            if (L >= c) return L;
        }
        while (on) on = walk_step<16>(q, k, i, j, lo, c);
    }
    if (bound && lo > 0 && i - c < lo && j - c >= 0) {
        const int jj = j - c;
        c += jj - bound[(long)(lo / strip - 1) * n + jj];
    } else if (wb && s0 > dlo && i - c < s0 && j - c >= 0) {
        c += (int)wb[dense_strip_offset(s0 >> 6) + (j - c)];
    }
    return c;
}

// strip boundaries of row bh when its pair walks use them (mode 2), else null
__device__ __forceinline__ const uint16_t* walk_bound_of(const PathArgs& a, int bh) {
    return a.o.dflag[bh] == 2 ? a.o.dbound + (long)bh * dense_row_entries(a.n) : nullptr;
}

__device__ __forceinline__ int owner_class(int cnt) {
    return cnt <= OWNER_SMALL ? 0 : cnt <= OWNER_MEDIUM ? 1 : 2;
}

// ---- walk-cost probe of one bigram pair (walk_probe_kernel below; pair_plan_kernel probes
// the small-class query owners of the rows it plans itself)
constexpr int WALK_EXACT = 64;
constexpr int WALK_COUNTED = 16;

// the run's exact length (its walk, once per run end)
__device__ __forceinline__ int probe_run(const int32_t* __restrict__ q,
                                         const int32_t* __restrict__ k, int i, int j, int dlo) {
    int c = i - 1 >= dlo ? 2 : 1;
    if (c == 2 && walk_step<4>(q, k, i, j, dlo, c)) {
        while (walk_step<16>(q, k, i, j, dlo, c)) {
        }
    }
    return c;
}

// query i's pair with key j of row bh: when the pair ends its diagonal run, the run's walk
// cost (runs of at least WALK_COUNTED labels) and, for runs of at least RUN_MIN labels in
// rows that list them, a run-list entry
__device__ __forceinline__ unsigned long long probe_pair(const PathArgs& a, int bh,
                                                         const int32_t* __restrict__ q,
                                                         const int32_t* __restrict__ k, int i,
                                                         int j, int dlo, bool next_reset,
                                                         bool listed) {
    const int n = a.n;
    const bool ends = i + 1 >= n || j + 1 >= n || next_reset || q[i + 1] != k[j + 1];
    if (!ends) return 0ull;
    const int lr = probe_run(q, k, i, j, dlo);
    if (lr >= RUN_MIN && listed) {
        const int slot = atomicAdd(&a.o.runcnt[bh], 1);
        if (slot < RUN_CAP) a.o.runs[(long)bh * RUN_CAP + slot] = make_int4(i - j, i, lr, 0);
    }
    const unsigned long long l = (unsigned long long)lr;
    return l >= WALK_COUNTED ? l * l / 2 : 0ull;
}

// Plan of the rows prepared in global memory (mode 0): one lane per owner (both sides,
// grid = 2 * B*H * ceil(N/64) items, one 64-owner chunk each): partner range by binary
// searches in the bigram orders, pair count per query row (pnb, by position), and the owner
// record staged in its row's class list (one atomic per wave and class).
__global__ __launch_bounds__(64 * WAVES) void pair_plan_kernel(PathArgs a) {
    const int n = a.n, lane = lane_id();
    const int per = (n + 63) / 64;
    const int item = xcd_work_item();
    const int side = item & 1;
    const int bh = (item >> 1) / per;
    if (bh >= a.B * a.H || a.o.mode[bh]) return;
    const long so = (long)bh * n;
    const int chunk = (item >> 1) - bh * per;
    const int t = chunk * 64 + lane;
    const bool own = t < n;
    const int tc = own ? t : n - 1;
    const int p = a.o.bpos[side][so + tc];
    int lo = 0, cnt = 0;
    if (own) {
        if (side == 0) partner_range<0>(a, bh, so, tc, p, lo, cnt);
        else partner_range<1>(a, bh, so, tc, p, lo, cnt);
        if (side == 0) a.pnb[so + p] = cnt;
    }
    const int cls = owner_class(cnt);
    // the walk-cost probe of this row's small-class query owners (walk_probe_kernel skips
    // them): their partners are at hand here, one lane per owner, at most OWNER_SMALL pairs
    if (side == 0 && own && cnt > 0 && cls == 0 && !pairless_mode(a.o.dflag[bh])) {
        const int32_t* kb = a.o.bpos[1] + so;
        const int32_t* q = a.iq + so;
        const int32_t* k = a.ik + so;
        const int dlo = walk_lo(a, so, p);
        const bool next_reset = p + 1 < n && walk_lo(a, so, p + 1) == p + 1;
        const bool listed = a.o.runs && !a.wlo && !a.dstart;
        unsigned long long cost = 0;
        for (int x = 0; x < cnt; ++x)
            cost += probe_pair(a, bh, q, k, p, kb[lo + x], dlo, next_reset, listed);
        if (cost) atomicAdd(&a.o.dcost[bh], cost);
    }
    const bool has = own && cnt > 0;
    const int4 rec = make_int4(bh, p, lo, cnt);
    int32_t* counts = a.o.bhcount[side] + (long)bh * 4;
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const unsigned long long m = __ballot(has && cls == c);
        if (!m) continue;
        int base = 0;
        if (lane == 0) base = atomicAdd(counts + c, __popcll(m));
        base = __shfl(base, 0);
        if (has && cls == c) {
            const int k = base + __popcll(m & below);
            if (c == 1) a.o.stage[side][1][so + k] = rec;
            else a.o.stage[side][0][so + (c == 0 ? k : n - 1 - k)] = rec;
        }
    }
}

hipError_t launch_pair_plan(const PathArgs& a, hipStream_t s) {
    const long chunks = ((a.n + 63) / 64) * (long)a.B * a.H;
    hipLaunchKernelGGL(pair_plan_kernel, dim3(grid_for(2 * chunks)), dim3(64 * WAVES), 0, s, a);
    return hipGetLastError();
}

// Owner lists: grid (B*H, 2 sides, slices); workgroup (bh, side, z) finds its row's offset in
// each class list (rows before it) and the class totals, then copies slice z of its staged
// records of each class (and, for query rows, their pair counts into pnb, whose other
// entries are zero).  Slices of a row split each class's records evenly, so long rows are
// copied by many workgroups instead of one.
constexpr int LIST_THREADS = 256;
constexpr int LIST_SLICE = 512;   // positions per slice of a row (the grid's z extent)
__global__ __launch_bounds__(LIST_THREADS) void owner_lists_kernel(PathArgs a) {
    __shared__ int s_red[LIST_THREADS / 64][8];
    const int bh = blockIdx.x, side = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int BH = a.B * a.H, n = a.n;
    const int32_t* cnt = a.o.bhcount[side];
    const int32_t* dense = a.o.dflag;  // dense rows' pairs belong to dism_dense.hip
    int before[3] = {0, 0, 0}, total[3] = {0, 0, 0};
    for (int r = tid; r < BH; r += LIST_THREADS) {
        const bool drop = pairless_mode(dense[r]);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const int v = drop ? 0 : cnt[(long)r * 4 + c];
            total[c] += v;
            if (r < bh) before[c] += v;
        }
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            before[c] += __shfl_xor(before[c], o);
            total[c] += __shfl_xor(total[c], o);
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            s_red[tid >> 6][c] = before[c];
            s_red[tid >> 6][4 + c] = total[c];
        }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        before[c] = 0;
        total[c] = 0;
        for (int w = 0; w < LIST_THREADS / 64; ++w) {
            before[c] += s_red[w][c];
            total[c] += s_red[w][4 + c];
        }
    }
    const int base[3] = {0, total[0], total[0] + total[1]};
    const long so = (long)bh * n;
    int4* own = a.o.own[side];
    const int z = blockIdx.z, slices = gridDim.z;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const int m = pairless_mode(dense[bh]) ? 0 : cnt[(long)bh * 4 + c];
        const int per = (m + slices - 1) / slices;
        const int k0 = z * per, k1 = k0 + per < m ? k0 + per : m;
        const int4* src = a.o.stage[side][c == 1 ? 1 : 0] + so;
        for (int k = k0 + tid; k < k1; k += LIST_THREADS) {
            const int4 rec = src[c == 2 ? n - 1 - k : k];
            own[base[c] + before[c] + k] = rec;
            if (side == 0) a.pnb[so + rec.y] = rec.w;  // pair count of the query row
        }
    }
    if (bh == 0 && z == 0 && tid < 3) a.o.ocount[4 * side + tid] = total[tid];
}

hipError_t launch_owner_lists(const PathArgs& a, hipStream_t s) {
    const unsigned slices = (unsigned)((a.n + LIST_SLICE - 1) / LIST_SLICE);
    hipLaunchKernelGGL(owner_lists_kernel, dim3((unsigned)(a.B * a.H), 2, slices),
                       dim3(LIST_THREADS), 0, s, a);
    return hipGetLastError();
}

// The rows the LDS-resident kernel can take (N <= PREP_N, unpacked, one label byte) run role
// 0 / role 1 of prepare_lds_kernel; the global-memory sort takes the others (its roles 0 /
// 1-2), deciding which from the labels as prepare_lds_kernel does.  Every kernel that decides
// writes the same row modes, so the halves may run on different streams.  The bigram half
// starts with its short kernels (sort and plan exit early on one-byte rows), so that on a
// busy device the long LDS kernel is the last to wait for free compute units.
static bool lds_rows(const PathArgs& pa) { return pa.n <= PREP_N && !pa.dstart; }

static SortArgs sort_args(const SortArgs& sa, const PathArgs& pa) {
    SortArgs b = sa;
    b.lds_rows = lds_rows(pa) ? 1 : 0;
    return b;
}

hipError_t launch_classify(const SortArgs& sa, hipStream_t s) {
    const int prefix = sa.prefix && sa.o.pxT ? 1 : 0;
    return launch_dense_classify(sa.lab[0], sa.lab[1], sa.BH, sa.n, sa.cls_n, prefix,
                                 sa.o.dflag, sa.o.dcost, sa.o.runcnt, s);
}

hipError_t launch_prepare_labels(const SortArgs& sa, const PathArgs& pa, hipStream_t s) {
    const SortArgs b = sort_args(sa, pa);
    // prepare_lds_kernel role 0 orders every row: in LDS, or in global memory for rows whose
    // labels differ in more than one byte
    hipError_t e = b.lds_rows ? launch_prepare_lds(b, 0, 1, s) : launch_msort_labels(b, s);
    return e != hipSuccess ? e : launch_ctab_balance(b, s);
}

hipError_t launch_prepare_pairs(const SortArgs& sa, const PathArgs& pa, hipStream_t s) {
    const SortArgs b = sort_args(sa, pa);
    hipError_t e;
    if (!b.lds_rows) {
        e = launch_msort_pairs(b, s);
        if (e == hipSuccess) e = launch_pair_plan(pa, s);
    } else {
        e = launch_sort(b, 1, 2, s);
        if (e == hipSuccess) e = launch_pair_plan(pa, s);
        if (e == hipSuccess) e = launch_prepare_lds(b, 1, 1, s);
    }
    if (e == hipSuccess) e = launch_owner_lists(pa, s);
    if (e == hipSuccess) e = launch_walk_probe(pa, s);
    return e != hipSuccess ? e : launch_dense_prepare(pa, s);
}

hipError_t launch_prepare(const SortArgs& sa, const PathArgs& pa, hipStream_t s) {
    const SortArgs b = sort_args(sa, pa);
    if (!b.lds_rows) {
        hipError_t e = launch_classify(sa, s);
        if (e == hipSuccess) e = launch_prepare_labels(sa, pa, s);
        return e != hipSuccess ? e : launch_prepare_pairs(sa, pa, s);
    }
    // one stream: the dense-row flags, both LDS roles in one grid (64-block roles side by
    // side), then the bigram sorts of the other rows, the plan, the owner lists and the dense
    // rows' list and boundaries
    hipError_t e = launch_classify(sa, s);
    if (e == hipSuccess) e = launch_prepare_lds(b, 0, 2, s);
    if (e == hipSuccess) e = launch_ctab_balance(b, s);
    if (e == hipSuccess) e = launch_sort(b, 1, 2, s);
    if (e == hipSuccess) e = launch_pair_plan(pa, s);
    if (e == hipSuccess) e = launch_owner_lists(pa, s);
    if (e == hipSuccess) e = launch_walk_probe(pa, s);
    return e != hipSuccess ? e : launch_dense_prepare(pa, s);
}

// Work of the persistent pair kernels of one side: items [0, i0) small class (16 owners
// each), [i0, i01) medium (4 owners), [i01, total) large (1 owner).
struct OwnerWork {
    int i0, i01, total, n[3], base[3];
};
template <int SIDE, int GS, int GM>
__device__ __forceinline__ OwnerWork owner_work(const PathArgs& a) {
    const int32_t* c = a.o.ocount + 4 * SIDE;
    OwnerWork w;
    w.n[0] = c[0];
    w.n[1] = c[1];
    w.n[2] = c[2];
    w.base[0] = 0;
    w.base[1] = w.n[0];
    w.base[2] = w.n[0] + w.n[1];
    w.i0 = (w.n[0] + 64 / GS - 1) / (64 / GS);
    w.i01 = w.i0 + (w.n[1] + 64 / GM - 1) / (64 / GM);
    w.total = w.i01 + w.n[2];
    return w;
}

// Owner of this lane's slot (G lanes per slot).
struct Slot {
    int bh, h, p, lo, cnt, maxcnt;
    bool hard;
    long so, row0;
};
template <int SIDE, int G>
__device__ __forceinline__ bool load_slot(const PathArgs& a, int base, int k0, int ncls,
                                          Slot& s) {
    const int sl = lane_id() / G;
    const int k = k0 + sl;
    const bool in = k < ncls;
    const int4 r = a.o.own[SIDE][base + (in ? k : ncls - 1)];
    const int b = r.x / a.H;
    s.bh = r.x;
    s.h = r.x - b * a.H;
    s.p = r.y;
    s.lo = r.z;
    // soft rows compute but write nothing (and walk unbounded: their carry boundary is
    // unset), off the dependent chain; the prepare's walk probe runs without row flags
    s.hard = a.hard ? a.hard[r.x] != 0 : true;
    s.cnt = in ? r.w : 0;
    s.so = (long)r.x * a.n;
    s.row0 = (long)b * a.n * a.H + s.h;
    int mx = s.cnt;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const int v = __shfl_xor(mx, o);
        mx = v > mx ? v : mx;
    }
    s.maxcnt = __builtin_amdgcn_readfirstlane(mx);
    return s.maxcnt > 0;
}

// Runs `item(G-tag, list base, first owner, class size)` for every item of side SIDE this
// wave strides over.
template <int G> struct Lanes { static constexpr int value = G; };
template <int SIDE, int GS, int GM, typename F>
__device__ __forceinline__ void for_owner_items(const PathArgs& a, F&& item) {
    static_assert(OWNER_SMALL <= GS && OWNER_MEDIUM <= GM, "owner classes must fit their lanes");
    const OwnerWork w = owner_work<SIDE, GS, GM>(a);
    const int stride = (int)gridDim.x * WAVES;
    for (int vi = (int)blockIdx.x * WAVES + wave_id_v(); vi < w.total; vi += stride) {
        if (vi < w.i0) item(Lanes<GS>{}, w.base[0], vi * (64 / GS), w.n[0]);
        else if (vi < w.i01) item(Lanes<GM>{}, w.base[1], (vi - w.i0) * (64 / GM), w.n[1]);
        else item(Lanes<64>{}, w.base[2], vi - w.i01, w.n[2]);
    }
}

// Pairwise tree ((t0 + t1) + (t2 + t3)) + ... over products t[d] = a[d] * b[d].
template <int N>
__device__ __forceinline__ float tree_dot(const float (&a)[N], const float (&b)[N]) {
    float t[N];
#pragma unroll
    for (int d = 0; d < N; ++d) t[d] = a[d] * b[d];
#pragma unroll
    for (int sz = 1; sz < N; sz *= 2)
#pragma unroll
        for (int g = 0; g < N; g += 2 * sz) t[g] = t[g] + t[g + sz];
    return t[0];
}

// ---------------------------------------------------------------------------------------
// forward, rows with pairs (after the label scan wrote y and the key count): sweep 1 finds
// the row shift m and the longest match (ties -> largest j), sweep 2 folds the corrections.
struct FinishLds {
    float cf[PAIR_SLOTS];
    float p[PAIR_SLOTS];
    int j[PAIR_SLOTS];
    unsigned m[64 / LANES_SMALL_MIN];
    unsigned long long key[64 / LANES_SMALL_MIN];
};

// N consecutive row elements of type T held as raw 32-bit words: bf16 pairs stay packed
// (unpacked at use) when N is even, otherwise the values are converted at load.
template <typename T, int N>
struct RawRow {
    static constexpr bool PACKED = sizeof(T) == 2 && N % 2 == 0;
    static constexpr int W = PACKED ? N / 2 : N;
    uint32_t w[W];
    __device__ __forceinline__ void load(const T* p) {
        if constexpr (PACKED) {
            load_words<W>(p, w);
        } else {
            float f[N];
            load_row<T, N>(p, f);
#pragma unroll
            for (int c = 0; c < N; ++c) w[c] = __float_as_uint(f[c]);
        }
    }
    __device__ __forceinline__ float at(int c) const {
        if constexpr (PACKED) return word_elem<T>(w, c);
        else return __uint_as_float(w[c]);
    }
};

// 64-bit shuffle (xor pattern)
__device__ __forceinline__ unsigned long long shfl_xor64(unsigned long long x, int m) {
    const int lo = __shfl_xor((int)(uint32_t)x, m), hi = __shfl_xor((int)(uint32_t)(x >> 32), m);
    return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
}

// ---------------------------------------------------------------------------------------
// Walk-cost probe (after the owner lists).  For every bigram pair that ends a diagonal run of
// matches ((i+1, j+1) does not continue it), the run's length l: exact up to WALK_EXACT
// labels, beyond that the largest offset 2^m at which the labels still match (within a factor
// 2 of a true run's length).  Per row, S += l^2 / 2, about the label comparisons that the
// run's pairs' walks would cost.  Rows with S > N^2 get strip boundaries (mode 2,
// dense_mode_kernel): their walks then stop within 64 rows (pair_length), so no row's walks
// cost more than O(N^2) in all.  The estimate only picks the method; lengths stay exact.
// Runs shorter than WALK_COUNTED are not counted: their pairs' walks take fewer than 16
// comparisons each, and a row that is not dense has at most about N^2/64 label-equal pairs,
// so together they cost under N^2/4; leaving them out keeps the per-row sum's atomics (one
// cache line for all rows) to the rare long runs.
// (WALK_EXACT, WALK_COUNTED, probe_run and probe_pair: before pair_plan_kernel)

template <int G>
__device__ __forceinline__ void probe_item(const PathArgs& a, int base, int k0, int ncls) {
    Slot s;
    if (!load_slot<0, G>(a, base, k0, ncls, s)) return;
    // small-class owners of rows planned in global memory were probed by pair_plan_kernel
    if (G == OWNER_SMALL && !a.o.mode[s.bh]) s.cnt = 0;
    const int n = a.n, sub = lane_id() % G;
    const int i = s.p;
    const int32_t* kb = a.o.bpos[1] + s.so;
    const int32_t* q = a.iq + s.so;
    const int32_t* k = a.ik + s.so;
    const int dlo = walk_lo(a, s.so, i);
    const bool next_reset = i + 1 < n && walk_lo(a, s.so, i + 1) == i + 1;
    const bool listed = a.o.runs && !a.wlo && !a.dstart;
    unsigned long long cost = 0;
    for (int c0 = 0; c0 < s.maxcnt; c0 += G) {
        const int kq = c0 + sub;
        if (kq < s.cnt) cost += probe_pair(a, s.bh, q, k, i, kb[s.lo + kq], dlo, next_reset, listed);
    }
#pragma unroll
    for (int o = G / 2; o >= 1; o >>= 1) cost += shfl_xor64(cost, o);
    if (sub == 0 && cost) atomicAdd(&a.o.dcost[s.bh], cost);
}

__global__ __launch_bounds__(64 * WAVES) void walk_probe_kernel(PathArgs a) {
    for_owner_items<0, OWNER_SMALL, OWNER_MEDIUM>(a, [&](auto g, int base, int k0, int ncls) {
        probe_item<decltype(g)::value>(a, base, k0, ncls);
    });
}

// The listed runs of each row sorted by (diagonal, end): one workgroup per row, a bitonic
// sort in LDS (lists of at most RUN_CAP records; a longer list is not used).
__global__ __launch_bounds__(1024) void run_sort_kernel(PathArgs a) {
    __shared__ unsigned long long s_k[RUN_CAP];
    __shared__ int s_l[RUN_CAP];
    const int bh = blockIdx.x, tid = threadIdx.x;
    const int cnt = a.o.runcnt[bh];
    if (cnt <= 1 || cnt > RUN_CAP) return;
    int4* runs = a.o.runs + (long)bh * RUN_CAP;
    int m = 1;
    while (m < cnt) m <<= 1;
    for (int x = tid; x < m; x += 1024) {
        if (x < cnt) {
            const int4 r = runs[x];
            s_k[x] = ((unsigned long long)(uint32_t)r.x << 32) | (uint32_t)r.y;
            s_l[x] = r.z;
        } else {
            s_k[x] = ~0ull;
            s_l[x] = 0;
        }
    }
    __syncthreads();
    for (int size = 2; size <= m; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int x = tid; x < m; x += 1024) {
                const int y = x ^ stride;
                if (y > x) {
                    const bool up = (x & size) == 0;
                    const unsigned long long kx = s_k[x], ky = s_k[y];
                    if ((kx > ky) == up) {
                        s_k[x] = ky;
                        s_k[y] = kx;
                        const int t = s_l[x];
                        s_l[x] = s_l[y];
                        s_l[y] = t;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int x = tid; x < cnt; x += 1024)
        runs[x] = make_int4((int)(s_k[x] >> 32), (int)(uint32_t)s_k[x], s_l[x], 0);
}

hipError_t launch_walk_probe(const PathArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(walk_probe_kernel, dim3(PAIR_GRID), dim3(64 * WAVES), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !a.o.runs || a.wlo || a.dstart) return e;
    hipLaunchKernelGGL(run_sort_kernel, dim3((unsigned)(a.B * a.H)), dim3(1024), 0, s, a);
    return hipGetLastError();
}

template <typename T, int R, int DV, int G>
__device__ __forceinline__ void finish_item(const PathArgs& a, int base, int k0, int ncls,
                                            FinishLds& S) {
    constexpr int CPL = DV >= G ? DV / G : 1;  // value columns per lane in phase B
    constexpr int GE = DV >= G ? G : DV;       // lanes of a slot holding columns
    Slot s;
    if (!load_slot<0, G>(a, base, k0, ncls, s)) return;
    const int n = a.n, lane = lane_id(), sl = lane / G, sub = lane % G;
    const int i = s.p, lo = s.lo, cnt = s.cnt;
    const int32_t* kb = a.o.bpos[1] + s.so;
    const int32_t* q = a.iq + s.so;
    const int32_t* k = a.ik + s.so;
    const int32_t* bnd = s.hard ? bound_of(a, s.bh) : nullptr;
    const uint16_t* wb = bnd ? nullptr : walk_bound_of(a, s.bh);
    const RunList rl = runs_of(a, s.bh);
    const float* lut = a.lut + (long)s.h * a.lut_stride;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const int cg = sub;
    const bool cols = cg < GE;
    const int col = (cols ? cg : 0) * CPL;
    // owner-side loads first (they depend only on the owner record)
    const float lut1 = lut[1];
    const float m0 = lut1 > 0.0f ? lut1 : 0.0f;
    float sqr[R];
    load_row<T, R>(sq + (s.row0 + (long)i * a.H) * R, sqr);
    const float* rec = a.prow + (s.so + i) * a.prow_stride;
    const int kc = __float_as_int(rec[PREC_CNT]);
    float y[CPL];
    load_row<float, CPL>(rec + PREC_Y + col, y);
    float dp = 0.0f, corr[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) corr[c] = 0.0f;
    float m;
    unsigned long long key;

    if (s.maxcnt <= G) {
        // one round: a lane per partner, the slot's pairs in flight together; the longest
        // match and the row shift by slot reductions, partner data to the column lanes by
        // shuffles, partner value rows loaded as soon as the partners are known
        const bool has = sub < cnt;
        const int j = kb[has ? lo + sub : 0];
        // partner rows loaded per batch, held as raw words (bf16 pairs unpacked at use, so a
        // batch holds twice the rows); the first batch is issued with the partners
        using RB_ = RawRow<T, CPL>;
        constexpr int UB = row_batch(RB_::W, 16);
        RB_ vr[UB];
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int jj = __shfl(j, sl * G + u);
            vr[u].load(v + (s.row0 + (long)jj * a.H) * DV + col);
        }
        float skr[R];
        load_row<T, R>(sk + (s.row0 + (long)j * a.H) * R, skr);
        const int L = has ? pair_length(q, k, i, j, bnd, a.strip, n, walk_lo(a, s.so, i), wb, rl) : 1;
        const float lw = lut[L];
        float mm = has && lw > m0 ? lw : m0;
        key = has ? (((unsigned long long)(unsigned)L << 32) | (unsigned)j) : 0ull;
#pragma unroll
        for (int o = G / 2; o >= 1; o >>= 1) {
            const float mo = __shfl_xor(mm, o);
            mm = mo > mm ? mo : mm;
            const unsigned long long ko = shfl_xor64(key, o);
            key = ko > key ? ko : key;
        }
        m = mm;
        const float p1 = exp2_fp32(lut1 - m);
        const float p = exp2_fp32(lw - m);
        float sdot = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sdot = __builtin_fmaf(sqr[r], skr[r], sdot);
        const float cf = (p - p1) * sdot;
        for (int u0 = 0; u0 < s.maxcnt; u0 += UB) {
            if (u0 > 0) {
#pragma unroll
                for (int u = 0; u < UB; ++u) {
                    const int jj = __shfl(j, sl * G + u0 + u);
                    vr[u].load(v + (s.row0 + (long)jj * a.H) * DV + col);
                }
            }
#pragma unroll
            for (int u = 0; u < UB; ++u) {
                const float pu = __shfl(p, sl * G + u0 + u), cfu = __shfl(cf, sl * G + u0 + u);
                if (u0 + u < cnt) {
                    dp = dp + pu;
#pragma unroll
                    for (int c = 0; c < CPL; ++c)
                        corr[c] = __builtin_fmaf(cfu, vr[u].at(c), corr[c]);
                }
            }
        }
    } else {
        // several rounds: sweep 1 (row shift, longest match) over all partners, then sweep 2
        if (sub == 0) {
            S.m[sl] = __float_as_uint(m0);
            S.key[sl] = 0ull;
        }
        for (int c0 = 0; c0 < s.maxcnt; c0 += G) {
            const int kq = c0 + sub;
            if (kq < cnt) {
                const int j = kb[lo + kq];
                const int L = pair_length(q, k, i, j, bnd, a.strip, n, walk_lo(a, s.so, i), wb, rl);
                const float lw = lut[L];
                if (lw > m0) atomicMax(&S.m[sl], __float_as_uint(lw));
                atomicMax(&S.key[sl], ((unsigned long long)(unsigned)L << 32) | (unsigned)j);
            }
        }
        m = __uint_as_float(S.m[sl]);
        key = S.key[sl];
        const float p1 = exp2_fp32(lut1 - m);
        float* cf_s = S.cf + sl * G;
        float* p_s = S.p + sl * G;
        int* j_s = S.j + sl * G;
        for (int c0 = 0; c0 < s.maxcnt; c0 += G) {
            // phase A: pair (slot, c0 + sub)
            const int kq = c0 + sub;
            if (kq < cnt) {
                const int j = kb[lo + kq];
                const int L = pair_length(q, k, i, j, bnd, a.strip, n, walk_lo(a, s.so, i), wb, rl);
                const float p = exp2_fp32(lut[L] - m);
                float skr[R];
                load_row<T, R>(sk + (s.row0 + (long)j * a.H) * R, skr);
                float sdot = 0.0f;
#pragma unroll
                for (int r = 0; r < R; ++r) sdot = __builtin_fmaf(sqr[r], skr[r], sdot);
                cf_s[sub] = (p - p1) * sdot;
                p_s[sub] = p;
                j_s[sub] = j;
            }
            // phase B: the slot folds its round's pairs in order, lane = column group cg
            const int nv = cnt - c0 < G ? cnt - c0 : G;
            if (cols) {
                constexpr int HB = row_batch(CPL, 4);
                for (int h0 = 0; h0 < nv; h0 += HB) {
                    float vr[HB][CPL];
#pragma unroll
                    for (int u = 0; u < HB; ++u) {
                        const int jj = j_s[h0 + u < nv ? h0 + u : nv - 1];
                        load_row<T, CPL>(v + (s.row0 + (long)jj * a.H) * DV + col, vr[u]);
                    }
#pragma unroll
                    for (int u = 0; u < HB; ++u) {
                        if (h0 + u < nv) {
                            dp = dp + p_s[h0 + u];
                            const float cf = cf_s[h0 + u];
#pragma unroll
                            for (int c = 0; c < CPL; ++c)
                                corr[c] = __builtin_fmaf(cf, vr[u][c], corr[c]);
                        }
                    }
                }
            }
        }
    }
    if (s.hard && cnt > 0 && cols) {
        const float p1 = exp2_fp32(lut1 - m);
        const float den = (exp2_fp32(-m) + (float)(kc - cnt) * p1) + dp;
        const float rden = 1.0f / den;
        const long orow = s.row0 + (long)i * a.H;
        if (a.out_dtype == DTYPE_F32) {
            float* o = reinterpret_cast<float*>(a.out) + orow * DV + col;
#pragma unroll
            for (int c = 0; c < CPL; ++c) o[c] = __builtin_fmaf(p1, y[c], corr[c]) * rden;
        } else {
            uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + orow * DV + col;
            if constexpr (CPL == 1) {
                o[0] = (uint16_t)f32_to_bf16_bits(__builtin_fmaf(p1, y[0], corr[0]) * rden);
            } else {
#pragma unroll
                for (int c = 0; c < CPL; c += 2) {
                    const uint32_t w0 =
                        f32_to_bf16_bits(__builtin_fmaf(p1, y[c], corr[c]) * rden);
                    const uint32_t w1 =
                        f32_to_bf16_bits(__builtin_fmaf(p1, y[c + 1], corr[c + 1]) * rden);
                    reinterpret_cast<uint32_t*>(o)[c / 2] = w0 | (w1 << 16);
                }
            }
        }
        if (cg == 0) {
            a.lse2[s.so + i] = m + log2_fp32(den);
            if (a.lmax) a.lmax[s.so + i] = (int)(key >> 32);
            if (a.jarg) a.jarg[s.so + i] = (int)(key & 0xffffffffu);
        }
    }
}

template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void pairs_finish_kernel(PathArgs a) {
    __shared__ FinishLds s_all[WAVES];
    FinishLds& S = s_all[wave_id_v()];
    constexpr int GS = lanes_small(DV, false), GM = lanes_medium(DV);
    for_owner_items<0, GS, GM>(a, [&](auto g, int base, int k0, int ncls) {
        finish_item<T, R, DV, decltype(g)::value>(a, base, k0, ncls, S);
    });
}

// Rows and keys: the DV-dot e = dO_i . v_j of each pair is taken in phase B, where the slot's
// lanes hold column groups: each lane's CPL contiguous columns as a pairwise tree of
// products, then the pairwise tree over the slot's lanes (group_sum) -- together the
// pairwise tree ((t0 + t1) + (t2 + t3)) + ... over all DV products t[d] = dO_i[d] * v_j[d].

// ---------------------------------------------------------------------------------------
// backward, query rows: row corrections [cdq[R], cu, cvv, cw, cz].
template <int R>
struct RowsLds {
    float f[PAIR_SLOTS][4];  // dp, s, av, j (bits)
    float sk[PAIR_SLOTS][R];
};

template <typename T, int R, int DV, int G>
__device__ __forceinline__ void rows_item(const PathArgs& a, int base, int k0, int ncls,
                                          RowsLds<R>& S) {
    constexpr int RL = (R + G - 1) / G;        // readout rows per lane in phase B
    constexpr int CPL = DV >= G ? DV / G : 1;  // value columns per lane in phase B
    constexpr int GE = DV >= G ? G : DV;       // lanes of a slot holding columns
    Slot s;
    if (!load_slot<0, G>(a, base, k0, ncls, s)) return;
    const int n = a.n, lane = lane_id(), sl = lane / G, sub = lane % G;
    const int i = s.p, lo = s.lo, cnt = s.cnt;
    const int32_t* kb = a.o.bpos[1] + s.so;
    const int32_t* q = a.iq + s.so;
    const int32_t* k = a.ik + s.so;
    const int32_t* bnd = s.hard ? bound_of(a, s.bh) : nullptr;
    const uint16_t* wb = bnd ? nullptr : walk_bound_of(a, s.bh);
    const RunList rl = runs_of(a, s.bh);
    const float* lut = a.lut + (long)s.h * a.lut_stride;
    const float* glut = a.dlut + (long)s.h * a.lut_stride;
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);

    const float l2 = a.lse2[s.so + i];
    const float cc = glut[i - doc_start(a, i) + 1];
    const float P1 = exp2_fp32(lut[1] - l2);
    const float q1 = P1 * (glut[1] - cc);
    const long qr = s.row0 + (long)i * a.H;
    const int col = (sub < GE ? sub : 0) * CPL;
    float sqr[R], dor[CPL];
    load_row<T, R>(sq + qr * R, sqr);
    load_row<T, CPL>(dout + qr * DV + col, dor);
    float cdq[RL], cu = 0.0f, cvv = 0.0f, cw = 0.0f, cz = 0.0f;
#pragma unroll
    for (int x = 0; x < RL; ++x) cdq[x] = 0.0f;
    const int sb = sl * G;

    if (s.maxcnt <= G) {
        // one round (see finish_item): partner value rows issued with the partners
        const bool has = sub < cnt;
        const int j = kb[has ? lo + sub : 0];
        constexpr int UB = row_batch(CPL, 16);
        float vr[UB][CPL];
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int jj = __shfl(j, sb + u);
            load_row<T, CPL>(v + (s.row0 + (long)jj * a.H) * DV + col, vr[u]);
        }
        float skr[R];
        load_row<T, R>(sk + (s.row0 + (long)j * a.H) * R, skr);
        const int L = has ? pair_length(q, k, i, j, bnd, a.strip, n, walk_lo(a, s.so, i), wb, rl) : 1;
        float sdot = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sdot = __builtin_fmaf(sqr[r], skr[r], sdot);
        const float p = exp2_fp32(lut[L] - l2);
        const float dpv = p - P1;
        const float av = p * (glut[L] - cc) - q1;
#pragma unroll
        for (int r = 0; r < R; ++r) S.sk[sb + sub][r] = skr[r];
        for (int u0 = 0; u0 < s.maxcnt; u0 += UB) {
            if (u0 > 0) {
#pragma unroll
                for (int u = 0; u < UB; ++u) {
                    const int jj = __shfl(j, sb + u0 + u);
                    load_row<T, CPL>(v + (s.row0 + (long)jj * a.H) * DV + col, vr[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < UB; ++u) {
                const float e = group_sum<GE>(tree_dot<CPL>(dor, vr[u]));
                const int src = sb + u0 + u;
                const float dpu = __shfl(dpv, src), su = __shfl(sdot, src), avu = __shfl(av, src);
                if (u0 + u < cnt) {
                    const float de = dpu * e;
#pragma unroll
                    for (int x = 0; x < RL; ++x) {
                        const int r = sub + G * x;
                        if (r < R) cdq[x] = __builtin_fmaf(de, S.sk[src][r], cdq[x]);
                    }
                    cu = __builtin_fmaf(dpu * su, e, cu);
                    cvv = cvv + avu;
                    cw = __builtin_fmaf(avu, su * e, cw);
                    cz = cz + dpu;
                }
            }
        }
    } else
    for (int c0 = 0; c0 < s.maxcnt; c0 += G) {
        const int kq = c0 + sub;
        if (kq < cnt) {
            const int j = kb[lo + kq];
            const int L = pair_length(q, k, i, j, bnd, a.strip, n, walk_lo(a, s.so, i), wb, rl);
            float skr[R];
            load_row<T, R>(sk + (s.row0 + (long)j * a.H) * R, skr);
            float sdot = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) sdot = __builtin_fmaf(sqr[r], skr[r], sdot);
            const float p = exp2_fp32(lut[L] - l2);
            float* f = S.f[sb + sub];
            f[0] = p - P1;
            f[1] = sdot;
            f[2] = p * (glut[L] - cc) - q1;
            f[3] = __int_as_float(j);
#pragma unroll
            for (int r = 0; r < R; ++r) S.sk[sb + sub][r] = skr[r];
        }
        const int nv = cnt - c0 < G ? cnt - c0 : G;
        constexpr int HB = row_batch(CPL, 4);
        for (int h0 = 0; h0 < s.maxcnt - c0 && h0 < G; h0 += HB) {
            float vr[HB][CPL];
#pragma unroll
            for (int u = 0; u < HB; ++u) {
                const int hu = h0 + u < nv ? h0 + u : (nv > 0 ? nv - 1 : 0);
                const int j = __float_as_int(S.f[sb + hu][3]);
                load_row<T, CPL>(v + (s.row0 + (long)(nv > 0 ? j : i) * a.H) * DV + col,
                                 vr[u]);
            }
#pragma unroll
            for (int u = 0; u < HB; ++u) {
                const float e = group_sum<GE>(tree_dot<CPL>(dor, vr[u]));
                if (h0 + u < nv) {
                    const float* f = S.f[sb + h0 + u];
                    const float dpv = f[0], sdot = f[1], av = f[2];
                    const float de = dpv * e;
#pragma unroll
                    for (int x = 0; x < RL; ++x) {
                        const int r = sub + G * x;
                        if (r < R) cdq[x] = __builtin_fmaf(de, S.sk[sb + h0 + u][r], cdq[x]);
                    }
                    cu = __builtin_fmaf(dpv * sdot, e, cu);
                    cvv = cvv + av;
                    cw = __builtin_fmaf(av, sdot * e, cw);
                    cz = cz + dpv;
                }
            }
        }
    }
    if (s.hard && cnt > 0) {
        float* rec = a.prow + (s.so + i) * a.prow_stride;
#pragma unroll
        for (int x = 0; x < RL; ++x) {
            const int r = sub + G * x;
            if (r < R) rec[r] = cdq[x];
        }
        if (sub == 0) {
            rec[R] = cu;
            rec[R + 1] = cvv;
            rec[R + 2] = cw;
            rec[R + 3] = cz;
        }
    }
}

// No occupancy target: at 4 waves/SIMD (128 VGPRs) the 16-label walk steps and the run-list
// lookups spill 356 bytes per lane, 220 MB of scratch writes per launch at configs[2]
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void pairs_rows_kernel(PathArgs a) {
    __shared__ RowsLds<R> s_all[WAVES];
    RowsLds<R>& S = s_all[wave_id_v()];
    constexpr int GS = lanes_small(DV, false), GM = lanes_medium(DV);
    for_owner_items<0, GS, GM>(a, [&](auto g, int base, int k0, int ncls) {
        rows_item<T, R, DV, decltype(g)::value>(a, base, k0, ncls, S);
    });
}

// ---------------------------------------------------------------------------------------
// backward keys: adds the bigram-pair corrections to dSK and dV written by the key scan.
template <int R>
struct KeysLds {
    float dp[PAIR_SLOTS];
    float s[PAIR_SLOTS];
    int i[PAIR_SLOTS];
    float sq[PAIR_SLOTS][R];
};

template <typename T, int R, int DV, int G>
__device__ __forceinline__ void keys_item(const PathArgs& a, int base, int k0, int ncls,
                                          KeysLds<R>& S) {
    constexpr int CPL = DV >= G ? DV / G : 1;
    constexpr int GE = DV >= G ? G : DV;
    constexpr int RL = (R + G - 1) / G;
    Slot s;
    if (!load_slot<1, G>(a, base, k0, ncls, s)) return;
    const int n = a.n, lane = lane_id(), sl = lane / G, sub = lane % G;
    const int j = s.p, lo = s.lo, cnt = s.cnt;
    const int32_t* qb = a.o.bpos[0] + s.so;
    const int32_t* q = a.iq + s.so;
    const int32_t* k = a.ik + s.so;
    const int32_t* bnd = s.hard ? bound_of(a, s.bh) : nullptr;
    const uint16_t* wb = bnd ? nullptr : walk_bound_of(a, s.bh);
    const RunList rl = runs_of(a, s.bh);
    const float* lut = a.lut + (long)s.h * a.lut_stride;
    const float lut1 = lut[1];
    const T* sq = reinterpret_cast<const T*>(a.sq);
    const T* sk = reinterpret_cast<const T*>(a.sk);
    const T* v = reinterpret_cast<const T*>(a.v);
    const T* dout = reinterpret_cast<const T*>(a.dout);

    const long kr = s.row0 + (long)j * a.H;
    const bool cols = sub < GE;
    const int col = (cols ? sub : 0) * CPL;
    float skr[R], vj[CPL];
    load_row<T, R>(sk + kr * R, skr);
    load_row<T, CPL>(v + kr * DV + col, vj);
    float cdk[RL], cdv[CPL];
#pragma unroll
    for (int x = 0; x < RL; ++x) cdk[x] = 0.0f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) cdv[c] = 0.0f;
    const int sb = sl * G;
    // the key scan's dSK0 / dV0 of this key, read now and written back with the corrections
    float dk0[RL], dv0[CPL];
#pragma unroll
    for (int x = 0; x < RL; ++x) {
        const int r = sub + G * x;
        dk0[x] = a.dsk[kr * R + (r < R ? r : 0)];
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) dv0[c] = a.dv[kr * DV + col + c];

    if (s.maxcnt <= G) {
        // one round (see finish_item): partner dO rows issued with the partners
        const bool has = sub < cnt;
        const int i = qb[has ? lo + sub : 0];
        constexpr int UB = row_batch(CPL, 16);
        float dr[UB][CPL];
#pragma unroll
        for (int u = 0; u < UB; ++u) {
            const int ii = __shfl(i, sb + u);
            load_row<T, CPL>(dout + (s.row0 + (long)ii * a.H) * DV + col, dr[u]);
        }
        const float l2 = a.lse2[s.so + i];
        float sqr[R];
        load_row<T, R>(sq + (s.row0 + (long)i * a.H) * R, sqr);
        const int L = has ? pair_length(q, k, i, j, bnd, a.strip, n, walk_lo(a, s.so, i), wb, rl) : 1;
        const float p = exp2_fp32(lut[L] - l2);
        float sdot = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) sdot = __builtin_fmaf(sqr[r], skr[r], sdot);
        const float dpv = p - exp2_fp32(lut1 - l2);
#pragma unroll
        for (int r = 0; r < R; ++r) S.sq[sb + sub][r] = sqr[r];
        for (int u0 = 0; u0 < s.maxcnt; u0 += UB) {
            if (u0 > 0) {
#pragma unroll
                for (int u = 0; u < UB; ++u) {
                    const int ii = __shfl(i, sb + u0 + u);
                    load_row<T, CPL>(dout + (s.row0 + (long)ii * a.H) * DV + col, dr[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < UB; ++u) {
                const float e = group_sum<GE>(tree_dot<CPL>(dr[u], vj));
                const int src = sb + u0 + u;
                const float dpu = __shfl(dpv, src), su = __shfl(sdot, src);
                if (u0 + u < cnt) {
                    const float de = dpu * e, ds = dpu * su;
#pragma unroll
                    for (int x = 0; x < RL; ++x) {
                        const int r = sub + G * x;
                        if (r < R) cdk[x] = __builtin_fmaf(de, S.sq[src][r], cdk[x]);
                    }
#pragma unroll
                    for (int c = 0; c < CPL; ++c) cdv[c] = __builtin_fmaf(ds, dr[u][c], cdv[c]);
                }
            }
        }
    } else
    for (int c0 = 0; c0 < s.maxcnt; c0 += G) {
        const int kq = c0 + sub;
        if (kq < cnt) {
            const int i = qb[lo + kq];
            const int L = pair_length(q, k, i, j, bnd, a.strip, n, walk_lo(a, s.so, i), wb, rl);
            const float l2 = a.lse2[s.so + i];
            const float p = exp2_fp32(lut[L] - l2);
            float sqr[R];
            load_row<T, R>(sq + (s.row0 + (long)i * a.H) * R, sqr);
            float sdot = 0.0f;
#pragma unroll
            for (int r = 0; r < R; ++r) sdot = __builtin_fmaf(sqr[r], skr[r], sdot);
            S.dp[sb + sub] = p - exp2_fp32(lut1 - l2);
            S.s[sb + sub] = sdot;
            S.i[sb + sub] = i;
#pragma unroll
            for (int r = 0; r < R; ++r) S.sq[sb + sub][r] = sqr[r];
        }
        const int nv = cnt - c0 < G ? cnt - c0 : G;
        constexpr int HB = row_batch(CPL, 4);
        for (int h0 = 0; h0 < s.maxcnt - c0 && h0 < G; h0 += HB) {
            float dr[HB][CPL];
#pragma unroll
            for (int u = 0; u < HB; ++u) {
                const int hu = h0 + u < nv ? h0 + u : (nv > 0 ? nv - 1 : 0);
                const int ii = nv > 0 ? S.i[sb + hu] : j;
                load_row<T, CPL>(dout + (s.row0 + (long)ii * a.H) * DV + col, dr[u]);
            }
#pragma unroll
            for (int u = 0; u < HB; ++u) {
                const float e = group_sum<GE>(tree_dot<CPL>(dr[u], vj));
                if (h0 + u < nv) {
                    const float dpv = S.dp[sb + h0 + u];
                    const float de = dpv * e, ds = dpv * S.s[sb + h0 + u];
#pragma unroll
                    for (int x = 0; x < RL; ++x) {
                        const int r = sub + G * x;
                        if (r < R) cdk[x] = __builtin_fmaf(de, S.sq[sb + h0 + u][r], cdk[x]);
                    }
#pragma unroll
                    for (int c = 0; c < CPL; ++c) cdv[c] = __builtin_fmaf(ds, dr[u][c], cdv[c]);
                }
            }
        }
    }
    if (s.hard && cnt > 0) {
#pragma unroll
        for (int x = 0; x < RL; ++x) {
            const int r = sub + G * x;
            if (r < R) a.dsk[kr * R + r] = dk0[x] + cdk[x];
        }
        if (cols) {
            float* g = a.dv + kr * DV + col;
#pragma unroll
            for (int c = 0; c < CPL; ++c) g[c] = dv0[c] + cdv[c];
        }
    }
}

template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * WAVES) void pairs_keys_kernel(PathArgs a) {
    __shared__ KeysLds<R> s_all[WAVES];
    KeysLds<R>& S = s_all[wave_id_v()];
    constexpr int GS = lanes_small(DV, true), GM = lanes_medium(DV);
    for_owner_items<1, GS, GM>(a, [&](auto g, int base, int k0, int ncls) {
        keys_item<T, R, DV, decltype(g)::value>(a, base, k0, ncls, S);
    });
}

// ---------------------------------------------------------------------------------------
#define DISM_PAIRS_LAUNCHER(NAME, KERNEL)                                                     \
    template <typename T, int R, int DV>                                                      \
    static hipError_t NAME##_go(const PathArgs& a, hipStream_t s) {                           \
        hipLaunchKernelGGL((KERNEL<T, R, DV>), dim3(PAIR_GRID), dim3(64 * WAVES), 0, s, a);    \
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

DISM_PAIRS_LAUNCHER(pairs_finish, pairs_finish_kernel)
DISM_PAIRS_LAUNCHER(pairs_rows, pairs_rows_kernel)
DISM_PAIRS_LAUNCHER(pairs_keys, pairs_keys_kernel)

}  // namespace dism
