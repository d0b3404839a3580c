// dism_launch.h -- host-side launchers exported by the .hip translation units to the C-ABI
// layer (dism_capi.cpp).  Plain pointers and sizes only.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace dism {

enum { DTYPE_BF16 = 0, DTYPE_F32 = 1 };
constexpr int SCAN_ITEM = 64;   // label-order entries that seed one scan work item

// Orders of one call (dism_sort.hip), each (b,h) row at offset bh*N (bh*2N for the
// combined order):
//   corder/clab/ctab: the 2N entries e = 2p + s (s = 0 key, 1 query at position p) sorted by
//                     (label, position, s), their labels, and the runs of the last sorted
//                     digit, (label >> shift) & 255 ([B*H][257]).
//   bpos/blab/bplab/btab (side 0 queries, 1 keys): positions sorted by
//                     (label[p-1], label[p], position), label[-1] := 0, with the runs of
//                     (label[p-1] >> shift) & 255.
// The digits come from the union of both sides' labels, so all tables share one digit
// (for labels below 256 a run is one label).
struct Orders {
    int32_t* corder;
    int32_t* clab;
    int32_t* ctab;
    int32_t* bpos[2];
    int32_t* blab[2];
    int32_t* bplab[2];
    int32_t* btab[2];
    int32_t* shift;       // [B*H]
    // bigram-pair owners (dism_sort.hip / dism_pairs.hip), side 0 query rows, 1 keys: a
    // record {bh, position, first partner index in the other side's bigram order, partner
    // count} per owner with partners, by class (OWNER_SMALL / OWNER_MEDIUM bounds):
    //   stage[side][0]: per (b,h) row (N slots at bh*N): small class from the front, large
    //                   class from the back;  stage[side][1]: medium class from the front;
    //   bhcount[side]:  [B*H][4] records of each class per row;
    //   own[side]:      all records, classes consecutive ([small][medium][large]), rows in
    //                   order inside a class;  ocount[4*side + class]: class totals.
    //   mode[bh]:       1 when the row was prepared by the LDS-resident kernel (N <= PREP_N
    //                   and labels that differ in one byte), 0 for the global-memory path.
    int4* stage[2][2];
    int32_t* bhcount[2];
    int4* own[2];
    int32_t* ocount;      // [8]
    int32_t* mode;        // [B*H]
    int32_t* onebyte;     // [B*H] 1 when the row's labels differ in at most one byte (shift)
    // multi-block sort (dism_msort.hip): digit counts [3*B*H][256][MSORT_SEGMENTS] (the
    // combined order's rows, then the bigram orders' rows), per-row partial label-bit masks
    // [B*H][32], then per-row digit lists [B*H][8]
    int32_t* mcount;
    int32_t* mdig;
    // dense rows (dism_dense.hip): per-row mode [B*H] (1: the row's bucketed label
    // collisions exceed N^2/64; 2: not dense, but its bigram walks would be long), the rows
    // of each kind ascending and their counts, and the 16-bit boundary rows L[64s - 1, j],
    // j < 64s, of every 64-row query strip s >= 1 of the rows of modes 1 and 2
    // ([B*H][dense_row_entries(N)], only when N <= DENSE_MAX_N)
    int32_t* dflag;       // row mode: 0 sparse, 1 dense, 2 sparse with strip-bounded walks,
                          // 3 dense level row (dism_levels.hip), 4 dense prefix row
                          // (dism_prefix.hip)
    int32_t* dlist;       // mode-1 rows, then (at dlist + B*H) the rows of modes 1 and 2, then
                          // (at dlist + 2*B*H) the mode-3 rows, (at dlist + 3*B*H) the mode-4
    int32_t* dcount;      // [0]: mode-1 rows, [1]: rows of modes 1 and 2, [2]: mode-3 rows,
                          // [3]: mode-4 rows
    uint16_t* dbound;
    unsigned long long* dcost;  // [B*H] walk-cost estimate of the probe (dism_pairs.hip)
    // long runs (dism_pairs.hip): per row, the run ends (diagonal i - j, end query i, exact
    // length) of the diagonal match runs of at least RUN_MIN labels, as the walk probe finds
    // them ([B*H][RUN_CAP] records, count in runcnt[B*H], cleared by the classification);
    // a pair walk that reaches RUN_MIN labels takes its length from its run's end.  Only for
    // calls without resets or documents.
    int4* runs;
    int32_t* runcnt;
    // level rows (mode 3, dism_levels.hip): dense rows whose sums are taken per match length.
    // Null unless N <= LEVEL_MAX_N and R * DV <= LEVEL_RDV.  Per (b,h) row:
    //   lvent  [LEVEL_MAX][2N]     level l's kept entries in list order (at (l - 1) 2N):
    //                              entry e = 2p + s in the low LEVEL_EBITS bits, a query's
    //                              count of keys before it in its group above them,
    //                              LEVEL_START on a group's first entry
    //   lvlc   [LEVEL_MAX + 2]     kept entries per level (per-level list construction)
    //   lvlf   [LEVEL_MAX + 1][N]  per level and position: 1 query kept, 2 with a key before
    //                              it, 4 key kept (per-level list construction)
    //   lvlk   [LEVEL_MAX][N]      per level: a query's last key before it in its group
    //   lvmeta [LEVEL_META]        level count, then off[0..LEVEL_MAX] (level l at
    //                              [off[l-1], off[l])), then segbase[0..LEVEL_MAX] (level l's
    //                              first segment of LEVEL_SEG entries)
    //   lvq    [N]                 per position {longest match Lq, its last key, kept levels
    //                              of the query, kept levels of the key}
    //   lvqidx / lvkidx [LEVEL_MAX][N]  index of query / key position p in level l's list
    //                              (written by the segment walks; valid for l up to the
    //                              position's kept level count)
    //   lvF, lvFk [level_segs(N)]  per segment: bit 0 a group starts in it, bit 1 at its first
    //                              entry (written by the forward / query-row and the key
    //                              chains, which may run concurrently)
    //   lvP    [level_segs(N)][R*DV]  forward segment totals T_s ([r][d])
    //   lvQ    [level_segs(N)][R*DV]  key-side segment totals U_s ([d][r])
    //   lvY    [LEVEL_BUDGET * N][DV]  per list entry: the forward's y_l of a query, the
    //                              backward's dv_l of a key
    //   lvZ    [LEVEL_BUDGET * N][R]   the backward's z_l of a query
    //   lvK    [LEVEL_BUDGET * N][R]   the backward's dk_l of a key
    int32_t* lvent;
    int32_t* lvlc;
    uint8_t* lvlf;
    uint16_t* lvlk;
    int32_t* lvmeta;
    int4* lvq;
    uint16_t* lvqidx;
    uint16_t* lvkidx;
    uint8_t* lvF;
    uint8_t* lvFk;
    float* lvP;
    float* lvQ;
    float* lvY;
    float* lvZ;
    float* lvK;
    // prefix rows (mode 4, dism_prefix.hip): dense rows in which every label has one
    // predecessor label, so every valid pair's match runs to the key's row start.  Per (b,h)
    // row, per segment s of PREFIX_SEG entries of the combined order ([px_segs(N)]):
    //   pxT, pxB [..][R*DV]  the forward's / query side's weighted key sums of the segment's
    //                        last group piece ([r][d]), overwritten by the chain with the
    //                        state before the segment (pxB: the d ln W / d tau weighted ones)
    //   pxU      [..][R*DV]  the key side's query sums of the first piece, then the state
    //                        after the segment
    //   pxS      [..]        {M, S, SG, (last key + 1) | PX_HAS | PX_RESET} per segment
    //   pxR      [..]        the state before the segment {mu, PS, PSG, last key}
    //   pxK      [..]        key side {lambda, has | restart << 1}
    //   pxKR     [..]        the state after the segment {nu, has}
    // Null unless N <= DENSE_MAX_N.
    float* pxT;
    float* pxB;
    float* pxU;
    float4* pxS;
    float4* pxR;
    float2* pxK;
    float2* pxKR;
    int32_t* pxE;     // [..][2N] a padded prefill row's list (entries of its real positions)
    int32_t* pxL;     // [..][2N] their labels
};
constexpr int LEVEL_MAX_N = 4096;   // longest level row (16-bit list indices and counts)
constexpr int LEVEL_MAX = 32;       // most levels (longest match) of a level row
constexpr int LEVEL_BUDGET = 16;    // kept entries per position over all levels
constexpr int LEVEL_SEG = 32;       // list entries per segment
constexpr int LEVEL_RDV = 512;      // largest R * DV of a level row
constexpr int LEVEL_START = 0x40000000;
constexpr int LEVEL_EBITS = 13;     // entry e < 2 LEVEL_MAX_N
constexpr int LEVEL_EMASK = (1 << LEVEL_EBITS) - 1;
constexpr int LEVEL_META = 2 * LEVEL_MAX + 4;
__host__ __device__ inline long level_segs(long n) {
    return (long)LEVEL_BUDGET * n / LEVEL_SEG + LEVEL_MAX;
}

// row modes computed whole by the dense, level or prefix kernels: no bigram-pair plan (the
// prepare's role 1 skips them, so their staged owner records and counts are not written)
__host__ __device__ inline bool pairless_mode(int m) { return m == 1 || m == 3 || m == 4; }

constexpr int PREFIX_SEG = 64;       // combined-order entries per prefix-row segment
__host__ __device__ inline int px_segs(int n) { return (2 * n + PREFIX_SEG - 1) / PREFIX_SEG; }

constexpr int DENSE_MAX_N = 65536;   // longest row of the dense path (16-bit lengths)
constexpr int RUN_MIN = 64;          // runs at least this long are listed (walks stop there)
constexpr int RUN_CAP = 4096;        // listed runs per row (more: the walks run in full)
constexpr int DENSE_BUCKETS = 4096;  // label buckets of the classification
__host__ __device__ inline long dense_strip_offset(int s) { return 32L * s * (s - 1); }
__host__ __device__ inline long dense_row_entries(int n) {
    const int q = (n + 63) / 64;
    return dense_strip_offset(q);
}

constexpr int PREP_N = 16384;     // longest row of the LDS-resident prepare kernel
constexpr int MSORT_SEGMENTS = 32;  // most workgroups per row of the multi-block sort
constexpr int OWNER_SMALL = 4;    // partner counts <= 4: 16 owners per wave, 4 lanes each
constexpr int OWNER_MEDIUM = 16;  // <= 16: 4 owners per wave, 16 lanes each; more: 1 per wave

struct SortArgs {
    const int32_t* lab[2];  // iq, ik  [B*H*N]
    long BH;
    int n;
    int32_t* tmp[3];        // scratch: [B*H*2N] combined, [B*H*N] per bigram side
    int32_t* pnb;           // [B*H*N] bigram pair count per query row (LDS-resident prepare)
    Orders o;
    int role_base;          // first role of a launch (blockIdx.y + role_base)
    int lds_rows;           // rows with one label byte go to prepare_lds_kernel (sort skips them)
    int cls_n;              // positions the dense-row classification counts (0: all n)
    int prefix;             // 1: dense rows may become prefix rows (fixed-length rows, no
                            // resets or documents; o.pxT set)
};

// Per query row record (prow, valid when the row's bigram pair count pnb > 0):
//   forward:  [-, key count, -, ..., y[DV] at PREC_Y] (y: the row's length-1 readout)
//   backward: [cdq[R], cu, cvv, cw, cz]
enum { PREC_CNT = 1, PREC_Y = 8 };

// Everything the pair and scan kernels of the hard core read or write.
struct PathArgs {
    int B, H, n;
    const int32_t* iq;       // [B,H,N]
    const int32_t* ik;
    const uint8_t* hard;     // [B*H]
    const float* lut;        // [H, lut_stride] log2 weights
    const float* dlut;       // [H, lut_stride] d ln W / d tau (backward)
    long lut_stride;
    const int32_t* bound;    // composed boundary [B,H,(N-1)/strip,N] or null
    int strip;
    Orders o;
    const void* sq;          // [B,N,H,R]  bf16 | f32
    const void* sk;
    const void* v;           // [B,N,H,DV]
    const void* dout;        // [B,N,H,DV] (backward)
    void* out;               // [B,N,H,DV] bf16 (out_dtype 0) or f32 (1)
    int out_dtype;
    float* lse2;             // [B,H,N] written by the forward, read by the backward
    int32_t* lmax;           // [B,H,N] nullable
    int32_t* jarg;           // [B,H,N] nullable
    int32_t* pnb;            // [B*H*N] bigram pair count per query row
    float* prow;             // [B*H*N][prow_stride]
    int prow_stride;
    float* dsq;              // [B,N,H,R] fp32
    float* dsk;
    float* dv;               // [B,N,H,DV] fp32
    float* rowtau;           // [B,H,N]
    // packed layouts (B = 1, dism_packed.hip): start of each token's document, or null for
    // fixed-length rows.  Walks stop at the query's document start, the pair plan drops the
    // diagonal pair at a document start, and G[i+1] uses the document-local position.
    const int32_t* dstart;   // [N]
    // query resets (inference prefill): per query the last reset position at or before it;
    // walks from that query stop there.  [B*H*N] or null.
    const int32_t* wlo;
    // positions of each row the prepare's dense-row classification and level lists take (a
    // prefill's rows are padded after the real tokens); 0: all n
    int cls_n;
    // forward label scan: 0 = every row, pair counts from pnb; 1 = rows whose labels differ
    // in one byte (onebyte), with the pair counts computed in the scan (the plan may still be
    // running on another stream); 2 = the remaining rows, from pnb.  Phases 1/2 only for
    // fixed-length rows (dstart null).
    int fwd_phase;
};

// Outputs a packed call zeroes on soft training rows (null pointers are skipped).
struct PackedZero {
    const uint8_t* hard;     // [rows, H]
    long row_tokens, H, n;
    int R, DV;
    void* out;
    int out_dtype;
    float* lse2;
    int32_t* lmax;
    int32_t* jarg;
    float* dsq;
    float* dsk;
    float* dv;
    float* rowtau;
};

// Incremental decoder (dism_decode.hip): state sections of one caller-owned buffer and the
// tokens of one call.
constexpr int LIST_BLOCK = 64;  // key positions per block of a label's position list
struct DecodeArgs {
    int rows, H, cap, slots, bcap;
    int R, DV;
    // state (one caller-owned buffer, dism_capi.cpp: decoder layout)
    int32_t* meta;        // [rows][4] position, pool blocks used, last reset, error
    int32_t* qlab;        // [rows][cap]
    int32_t* klab;        // [rows][cap]
    void* skh;            // [rows][cap][R]
    void* vh;             // [rows][cap][DV]
    int32_t* slot_label;  // [rows][slots]
    int32_t* slot_cnt;    // [rows][slots] keys of the label (0: empty slot)
    int32_t* slot_last;   // [rows][slots]
    float* M;             // [rows][slots][R*DV]
    int32_t* slot_blocks; // [rows][slots][bcap]
    int32_t* pool;        // [rows][pool_blocks * 64]
    int32_t* scratch;     // [rows][cap] walk lengths of the current query's candidates
    int pool_blocks;
    // this call's tokens: n per row, inputs in the training layouts with N = n
    int n;
    const int32_t* iq;    // [B,H,n]
    const int32_t* ik;
    const uint8_t* reset; // [B,H,n] or null
    const void* sq;       // [B,n,H,R] (null for prime)
    const void* sk;
    const void* v;        // [B,n,H,DV]
    const float* lut;     // [H, lut_stride]
    long lut_stride;
    float* out;           // [B,n,H,DV] fp32, null for prime (keys only)
    float* lse2;          // [B,H,n] or null
};

hipError_t launch_decode(const DecodeArgs& a, int dtype, hipStream_t s);
hipError_t launch_pad_labels(const int32_t* src, long rows, long n, long npad, int32_t* dst,
                             hipStream_t s);
// keys-only state of a whole prompt of a.n tokens from its combined label order (rows of npad)
hipError_t launch_prime(const DecodeArgs& a, const Orders& o, int npad, int dtype,
                        hipStream_t s);
hipError_t launch_reset_starts(const uint8_t* reset, long rows, long n, int32_t* wlo,
                               hipStream_t s);

// x, vocab: bf16; list: caller scratch [1 + 2H + B*H*N] (count of fp64-rescored tokens, per
// head vocabulary statistics, the rescored tokens)
hipError_t launch_vocab_argmax(const void* x, const void* vocab, long vhs, int B, int N, int H,
                               int V, int D, int32_t* labels, int32_t* list, hipStream_t s);
hipError_t launch_sign_labels(const void* x, int dtype, long B, long N, long H, int d,
                              int32_t* out, hipStream_t s);
hipError_t launch_log_weights(const float* tau, int H, long stride, float* out, hipStream_t s);
hipError_t launch_dlog_weights(const float* tau, int H, long stride, float* out, hipStream_t s);
hipError_t launch_boundary(const int32_t* iq, const int32_t* ik, const uint8_t* hard, long BH,
                           int n, int strip, int composed, int fill_all, int32_t* out,
                           hipStream_t s);
hipError_t launch_chunk(const int32_t* summary, int32_t* out, long BH, long C, int n,
                        hipStream_t s);
hipError_t launch_tau_reduce(const float* rowtau, int B, int H, long n, float* dtau,
                             hipStream_t s);
hipError_t launch_fill_i32(int32_t* p, long count, int32_t value, hipStream_t s);
hipError_t launch_packed_docs(const int32_t* cu, int docs, long H, long n, int32_t* dstart,
                              int32_t* dindex, uint8_t* ones, hipStream_t s);
hipError_t launch_packed_tags(const int32_t* corder, const int32_t* clab,
                              const int32_t* dindex, int docs, long H, long n, int32_t* tq,
                              int32_t* tk, hipStream_t s);
hipError_t launch_packed_soft_zero(const PackedZero& z, hipStream_t s);
// Position orders and bigram-pair plans of a prepare call: the LDS-resident kernel for the
// rows it can take, the global-memory sort and plan for the others, then the owner lists.
hipError_t launch_prepare(const SortArgs& sa, const PathArgs& pa, hipStream_t s);
// the row modes' first step, the dense-row flags (dflag, and dcost cleared): both halves below
// read them, so it runs before either is launched
hipError_t launch_classify(const SortArgs& sa, hipStream_t s);
// the two independent halves of launch_prepare (after launch_classify): the combined label
// order (what the label scans need) and the bigram orders, pair plans and owner lists (what
// the pair kernels need)
hipError_t launch_prepare_labels(const SortArgs& sa, const PathArgs& pa, hipStream_t s);
hipError_t launch_prepare_pairs(const SortArgs& sa, const PathArgs& pa, hipStream_t s);
hipError_t launch_sort(const SortArgs& a, int role0, int roles, hipStream_t s);
// multi-block sorts (rows the LDS-resident kernel cannot take): the combined label order, and
// the bigram orders of both sides (each also lists the rows' digits, mode and shift)
hipError_t launch_msort_labels(const SortArgs& a, hipStream_t s);
hipError_t launch_msort_pairs(const SortArgs& a, hipStream_t s);
// only the combined label order (corder, clab, ctab) of every row, global-memory path (the
// rows' mode must be 0)
hipError_t launch_sort_labels(const SortArgs& a, hipStream_t s);
hipError_t launch_prepare_lds(const SortArgs& a, int role0, int roles, hipStream_t s);
// label-scan buckets of about 2N/256 entries for rows with multi-byte labels (after the
// combined label order)
hipError_t launch_ctab_balance(const SortArgs& a, hipStream_t s);
// The following return hipErrorInvalidValue for an unsupported (R, DV, dtype).
hipError_t launch_pair_plan(const PathArgs& a, hipStream_t s);
hipError_t launch_owner_lists(const PathArgs& a, hipStream_t s);
hipError_t launch_pairs_finish(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_scan_forward(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_pairs_rows(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_scan_rows(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_pairs_keys(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
// dense rows (dism_dense.hip): classification (before the label scans), the row list and the
// boundary rows (before the dense kernels), then the tile kernels for the flagged hard rows
// (prefix: dense rows may become prefix rows, mode 4; calls without resets or documents)
hipError_t launch_dense_classify(const int32_t* iq, const int32_t* ik, long BH, int n,
                                 int cls_n, int prefix, int32_t* dflag,
                                 unsigned long long* dcost, int32_t* runcnt, hipStream_t s);
hipError_t launch_walk_probe(const PathArgs& a, hipStream_t s);
// level lists of the dense rows that qualify (mode 1 -> 3; dism_sort.hip), before the row
// lists of launch_dense_prepare
hipError_t launch_level_prep(const PathArgs& a, hipStream_t s);
// level rows: forward (segment prefixes, then the readout), backward query rows, backward
// keys (dism_levels.hip); no-ops without level rows
hipError_t launch_level_forward(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_level_rows(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_level_keys(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
// prefix rows (classified by launch_dense_classify): forward (segment totals, chain, readout),
// backward query rows, backward keys (dism_prefix.h); no-ops without prefix rows
hipError_t launch_prefix_forward(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_prefix_rows(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_prefix_keys(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_dense_prepare(const PathArgs& a, hipStream_t s);
hipError_t launch_dense_forward(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_dense_rows(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_dense_keys(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_scan_keys(const PathArgs& a, int R, int DV, int dtype, hipStream_t s);

// ---------------------------------------------------------------------------------------
// Layout fingerprint of the argument structs the kernels take by value.  Every translation
// unit records the fingerprint it was compiled with (DISM_TU_LAYOUT); dism_layout_check()
// in dism_capi.cpp compares them on load and on the first call, so a library linked from
// objects compiled against different versions of these structs refuses to run instead of
// launching kernels that read their arguments at the wrong offsets.
static_assert(sizeof(void*) == 8 && sizeof(long) == 8, "LP64 host and device");
static_assert(sizeof(Orders) == 448, "Orders changed: update the size and the fingerprint");
static_assert(sizeof(SortArgs) == 528, "SortArgs changed: update the size and the fingerprint");
static_assert(sizeof(PathArgs) == 680, "PathArgs changed: update the size and the fingerprint");
static_assert(sizeof(PackedZero) == 112, "PackedZero changed: update the size");
static_assert(sizeof(DecodeArgs) == 216, "DecodeArgs changed: update the size");

constexpr unsigned long long fp_mix(unsigned long long h, unsigned long long v) {
    return (h ^ v) * 1099511628211ull;  // FNV-1a step over whole values
}
#define DISM_FP(S, f) h = fp_mix(h, offsetof(S, f))
constexpr unsigned long long layout_fingerprint() {
    unsigned long long h = 1469598103934665603ull;
    h = fp_mix(h, sizeof(Orders));
    h = fp_mix(h, sizeof(SortArgs));
    h = fp_mix(h, sizeof(PathArgs));
    h = fp_mix(h, sizeof(PackedZero));
    h = fp_mix(h, sizeof(DecodeArgs));
    DISM_FP(Orders, bpos); DISM_FP(Orders, shift); DISM_FP(Orders, stage);
    DISM_FP(Orders, ocount); DISM_FP(Orders, mcount); DISM_FP(Orders, dflag);
    DISM_FP(Orders, dlist); DISM_FP(Orders, dbound); DISM_FP(Orders, runs);
    DISM_FP(Orders, lvent); DISM_FP(Orders, lvK); DISM_FP(Orders, pxT);
    DISM_FP(Orders, pxE); DISM_FP(Orders, pxL);
    DISM_FP(SortArgs, BH); DISM_FP(SortArgs, n); DISM_FP(SortArgs, tmp);
    DISM_FP(SortArgs, pnb); DISM_FP(SortArgs, o); DISM_FP(SortArgs, role_base);
    DISM_FP(SortArgs, lds_rows); DISM_FP(SortArgs, cls_n); DISM_FP(SortArgs, prefix);
    DISM_FP(PathArgs, iq); DISM_FP(PathArgs, hard); DISM_FP(PathArgs, lut);
    DISM_FP(PathArgs, dlut); DISM_FP(PathArgs, lut_stride); DISM_FP(PathArgs, bound);
    DISM_FP(PathArgs, strip); DISM_FP(PathArgs, o); DISM_FP(PathArgs, sq);
    DISM_FP(PathArgs, sk); DISM_FP(PathArgs, v); DISM_FP(PathArgs, dout);
    DISM_FP(PathArgs, out); DISM_FP(PathArgs, out_dtype); DISM_FP(PathArgs, lse2);
    DISM_FP(PathArgs, lmax); DISM_FP(PathArgs, jarg); DISM_FP(PathArgs, pnb);
    DISM_FP(PathArgs, prow); DISM_FP(PathArgs, prow_stride); DISM_FP(PathArgs, dsq);
    DISM_FP(PathArgs, dsk); DISM_FP(PathArgs, dv); DISM_FP(PathArgs, rowtau);
    DISM_FP(PathArgs, dstart); DISM_FP(PathArgs, wlo); DISM_FP(PathArgs, cls_n);
    DISM_FP(PathArgs, fwd_phase);
    DISM_FP(PackedZero, R); DISM_FP(PackedZero, out); DISM_FP(PackedZero, rowtau);
    DISM_FP(DecodeArgs, meta); DISM_FP(DecodeArgs, pool_blocks); DISM_FP(DecodeArgs, n);
    DISM_FP(DecodeArgs, sq); DISM_FP(DecodeArgs, lut_stride); DISM_FP(DecodeArgs, lse2);
    return h;
}
#undef DISM_FP

}  // namespace dism

// One per translation unit: the fingerprint the unit was compiled with (read by
// dism_layout_check; an object compiled before a struct changed carries the old value).
#define DISM_TU_LAYOUT(tu) \
    extern "C" __attribute__((visibility("hidden"))) const unsigned long long \
        dism_layout_##tu = dism::layout_fingerprint();
