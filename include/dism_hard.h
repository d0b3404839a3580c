/*
 * dism_hard.h -- C ABI of the MI355X flash_dism hard (integer-label) core.
 *
 * Library: dism_amd/libdism_hip.so (gfx950).  Every entry point takes raw device pointers,
 * sizes and a HIP stream (passed as void*, a hipStream_t; NULL = default stream), enqueues
 * its kernels on that stream and returns without synchronising.  The caller allocates all
 * outputs; the library owns no device memory and keeps no mutable global state beyond a pool
 * of side streams (three events each, default priority) per device, one leased for the
 * duration of each entry point that forks (dism_hard_forward, dism_hard_backward and its
 * queries / keys stages), so calls on different streams or threads are independent.  Return value: 0 on success, otherwise
 * a DISM_ERR_* code with a thread-local message from dism_last_error().
 *
 * Layouts follow the reference: vectors BNHD ([B,N,H,R] / [B,N,H,DV], contiguous), labels
 * BHN int32, sequence hard flags [B,H] bool (uint8).  Vector dtype code: 0 = bf16, 1 = f32.
 * Supported readout dims R in {2,4,8,16,32}, DV in {32,64,128}.
 *
 * Each function names the reference interface it replaces (paths under cicuvc/dism).
 */
#ifndef DISM_HARD_H
#define DISM_HARD_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    DISM_OK = 0,
    DISM_ERR_INVALID = 1,     /* bad shape / size / pointer: reference raises RuntimeError */
    DISM_ERR_UNSUPPORTED = 2, /* (R, DV, dtype) combination not compiled */
    DISM_ERR_HIP = 3          /* HIP launch error */
};
enum { DISM_BF16 = 0, DISM_F32 = 1 };

/* Thread-local message of the last failing call on this thread ("" if none). */
const char* dism_last_error(void);
/* ABI version of this library. */
int32_t dism_abi_version(void);
/* DISM_OK when every translation unit of the library was compiled against the same layout of
 * the argument structs its kernels take by value; otherwise DISM_ERR_INVALID, naming the stale
 * units.  Every compute entry point performs the same check (once per process).  No
 * counterpart in the reference: its extension is one build-system target, this library is
 * linked from per-unit objects. */
int32_t dism_layout_check(void);

/* Sign binarizer, the label producer of this build: labels[b,h,n] = sum_k [x[b,n,h,k] > 0] 2^k
 * for k < d (d <= 30).  Replaces the vocabulary argmax label producer
 * dism_v3/python/flash_dism/emb_kernel.py:83-108 for hypercube codebooks (first-index tie
 * rule: x == 0 gives bit 0). */
int32_t dism_sign_labels(const void* x, int32_t dtype, int64_t B, int64_t N, int64_t H,
                         int32_t d, int32_t* labels, void* stream);

/* Vocabulary (codebook) labels: labels[b,h,n] = argmax_v sum_d x[b,n,h,d] * vocab[h,v,d] in
 * exact arithmetic, first index on ties; x bf16 [B,N,H,D], vocab bf16 [H,V,D] with head stride
 * vocab_head_stride elements (0 = one shared [V,D] table), D in {32,64,128}.  Matrix-core
 * scores with a certified error bound; tokens whose top-two margin is within the bound are
 * listed in scratch (caller-owned int32 [1 + 2H + B*H*N]: scratch[0] = how many) and
 * rescored in fp64 by a second kernel.  B*H*N < 2^31.  Replaces the
 * label output of the Triton interpolation (dism_v3/python/flash_dism/emb_kernel.py:83-108,
 * :155-156) and the oracle argmax (dism_v3/python/flash_dism/reference/dism_v3_ref.py:159-162);
 * the interpolated embeddings and LSE belong to the soft path. */
int32_t dism_vocab_labels(const void* x, const void* vocab, int64_t vocab_head_stride, int64_t B,
                          int64_t N, int64_t H, int64_t V, int32_t D, int32_t* labels,
                          int32_t* scratch, void* stream);

/* log2 geometric weight table lut[h, l] = log2 sum_{s=1..l} e^{s tau_h}, lut[h,0] = -1e6,
 * l in [0, max_length].  Replaces cu.hard_log_weights (dism_v3/src/host/hard_forward.cpp:11-23,
 * kernel dism_v3/src/hard_forward.cu:10-25). */
int32_t dism_hard_log_weights(const float* tau, int32_t H, int64_t max_length, float* lut,
                              void* stream);

/* Natural-tau derivative g[h, l] = d ln W_l / d tau_h, g[h,0] = 0, l < stride.
 * Replaces hard_dlog_weights_kernel (dism_v3/src/hard_backward.cu:8-23). */
int32_t dism_hard_dlog_weights(const float* tau, int32_t H, int64_t stride, float* dlut,
                               void* stream);

/* Strip-32 summaries int32 [B,H,(N-1)/32,N]: last mismatching key coordinate on the strip's
 * diagonal segment ending at (32c+31, j), -1 if none / non-causal / soft.
 * Replaces cu.hard_summary (dism_v3/src/host/hard_summary.cpp:11-72). */
int32_t dism_hard_summary(const int32_t* iq, const int32_t* ik, const uint8_t* hard, int64_t B,
                          int64_t H, int64_t N, int32_t* summary, void* stream);

/* Composition out[c,j] = max(s[c,j], out[c-1,j-32]) with non-causal -1, summaries of shape
 * [BH,(N-1)/32,N]; out may alias summary (in place).
 * Replaces cu.hard_chunk (dism_v3/src/host/hard_chunk.cpp:10-69). */
int32_t dism_hard_chunk(const int32_t* summary, int32_t* boundary, int64_t BH, int64_t N,
                        void* stream);

/* Composed boundaries in one pass for any strip height S: boundary[b,h,c,j] = j - L[cS+S-1, j]
 * on causal hard cells; non-causal/soft cells are -1 when fill_all != 0 and left untouched
 * otherwise.  S = 32 equals dism_hard_chunk(dism_hard_summary(.)) -- the fused replacement of
 * summarize_hard + hard_chunk_scan (dism_v3/python/flash_dism/summary.py:5-29). */
int32_t dism_hard_boundary(const int32_t* iq, const int32_t* ik, const uint8_t* hard, int64_t B,
                           int64_t H, int64_t N, int32_t strip, int32_t fill_all,
                           int32_t* boundary, void* stream);

/* Size in bytes of the caller-owned workspace for these dimensions (-1 for unsupported
 * dimensions, or B*H*N >= 2^31).  It holds the position orders of dism_hard_prepare
 * (combined label order of queries and keys, bigram position lists of each side), the
 * bigram-pair owner records, and one record per query row (partial readout in the forward,
 * row corrections in the backward); about 4*B*H*N*(DV + 48) bytes.
 * No reference counterpart: the reference keeps an O(B*H*N^2/32) int32 boundary instead. */
int64_t dism_hard_workspace_bytes(int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                  int32_t dtype);

/* Preparation into `workspace` (labels only; the vectors are validated, not read):
 *   - per (b,h): stable sorts giving the combined label order of the 2N query/key entries
 *     and the bigram order (label[p-1], label[p]) of the queries and of the keys;
 *   - per query row and per key: the range of its bigram partners (the pairs with match
 *     length >= 2), and the owners that have any, listed by partner-count class.
 * A workspace prepared once serves dism_hard_readout and the backward entry points for the
 * same labels.  Replaces the summary + chunk passes that precede the reference readout
 * (dism_v3/python/flash_dism/hard_forward.py:36-40). */
int32_t dism_hard_prepare(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, int64_t B, int64_t N, int64_t H,
                          int32_t R, int32_t DV, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* Allocation-free one-call forward: dism_hard_forward's outputs for the same inputs (bit for
 * bit), with its workspace in a device array inside the library instead of a caller buffer,
 * and every launch on `stream` (no side stream).  No reference counterpart: for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The array holds dism_hard_forward_noalloc_max_bytes() bytes (256 MiB) on every
 * device the library runs on, until the process ends; shapes whose
 * dism_hard_workspace_bytes exceeds it fail with DISM_ERR_INVALID.  All calls on one device
 * share the array: calls that overlap in time on one device (other streams, other threads)
 * race and must be serialized by the caller.  Calls no hipMalloc/hipFree. */
int64_t dism_hard_forward_noalloc_max_bytes(void);
int32_t dism_hard_forward_noalloc(const void* sq, const void* sk, const void* v, int32_t dtype,
                                  const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                                  const float* lut, int64_t lut_stride, int64_t B, int64_t N,
                                  int64_t H, int32_t R, int32_t DV, void* out, int32_t out_dtype,
                                  float* lse2, int32_t* lmax, int32_t* jarg, void* stream);

/* Row modes of a prepared workspace, [B*H] int32 to `modes` (device memory): 0 = sparse row
 * (label scans + bigram walks), 1 = dense row (the bucketed label collisions exceed N^2/64:
 * direct tile kernels), 2 = sparse row whose walks stop at 64-row strip boundaries (the walk
 * probe estimated their cost above N^2), 3 = dense level row (labels below 256, N <= 4096,
 * R*DV <= 512, at most 32 distinct match lengths: sums per match length), 4 = dense prefix
 * row (every label has one predecessor label, so every match runs to the key's row start:
 * prefix sums with per-key weights).  An introspection aid for tests and tuning; no
 * reference counterpart. */
int32_t dism_hard_row_modes(const void* workspace, int64_t workspace_bytes, int64_t B,
                            int64_t N, int64_t H, int32_t R, int32_t DV, int32_t* modes,
                            void* stream);

/* Hard readout on a prepared workspace: O [B,N,H,DV] (out_dtype bf16|f32) and lse2 [B,H,N]
 * fp32; optional lmax/jarg [B,H,N] int32 receive the longest match length per query and its
 * key (ties -> most recent key, -1 if none).  boundary may be NULL (lengths recomputed from
 * labels alone) or a composed boundary of strip height `strip`.  lut_stride >= N+1.  Soft
 * rows give zeros.  Vector pointers must be 16-byte aligned.
 * Replaces cu.hard_readout (dism_v3/src/host/hard_forward.cpp:25-113). */
int32_t dism_hard_readout(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                          const int32_t* boundary, int32_t strip, const float* lut,
                          int64_t lut_stride, int64_t B, int64_t N, int64_t H, int32_t R,
                          int32_t DV, void* workspace, int64_t workspace_bytes, void* out,
                          int32_t out_dtype, float* lse2, int32_t* lmax, int32_t* jarg,
                          void* stream);

/* dism_hard_prepare followed by dism_hard_readout, in one call with the same arguments as
 * dism_hard_readout (the workspace need not be prepared; it is on return, for the backward).
 * The row classification, the bigram half of the preparation and the readouts of dense,
 * level and prefix rows run on the calling thread's side stream (see dism_hard_backward),
 * overlapped with the label order and the length-1 label scan, and are joined back into
 * `stream` before the pair kernels.  Outputs are bit-identical to the two-call sequence.
 * Replaces the forward_hard chain summary -> chunk -> readout
 * (dism_v3/python/flash_dism/hard_forward.py:36-47). */
int32_t dism_hard_forward(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                          const int32_t* boundary, int32_t strip, const float* lut,
                          int64_t lut_stride, int64_t B, int64_t N, int64_t H, int32_t R,
                          int32_t DV, void* workspace, int64_t workspace_bytes, void* out,
                          int32_t out_dtype, float* lse2, int32_t* lmax, int32_t* jarg,
                          void* stream);

/* Hard backward on a workspace prepared by dism_hard_prepare for the same labels: dsq, dsk
 * [B,N,H,R], dv [B,N,H,DV], rowtau [B,H,N] (caller-owned scratch) and dtau [H], all fp32,
 * deterministic (no floating-point atomics).  lse2 is the forward's log2 normalizer;
 * lut/dlut share lut_stride >= N+1.  Runs the five stages below: the key chain (keys, key
 * pairs) on a side stream of the calling thread (default priority, created on first use and
 * kept; forked from and joined back into `stream`, so the call stays asynchronous and
 * capturable), the query-row chain (row pairs, queries, tau reduce) on `stream`.
 * Replaces cu.hard_backward (dism_v3/src/host/hard_backward.cpp:13-140). */
int32_t dism_hard_backward(const void* sq, const void* sk, const void* v, const void* dout,
                           int32_t dtype, const int32_t* iq, const int32_t* ik,
                           const uint8_t* hard, const int32_t* boundary, int32_t strip,
                           const float* lut, const float* dlut, int64_t lut_stride,
                           const float* lse2, int64_t B, int64_t N, int64_t H, int32_t R,
                           int32_t DV, void* workspace, int64_t workspace_bytes, float* dsq,
                           float* dsk, float* dv, float* rowtau, float* dtau, void* stream);

/* Stages of dism_hard_backward, callable separately in this order (same arguments as
 * above).  queries and keys run the kernels of dense, level and prefix rows on a leased side
 * stream beside their label scan and join it back before returning.  Together they replace the hard_dlog_weights / hard_backward /
 * hard_tau_reduce launch sequence of dism_v3/src/host/hard_backward.cpp:242-252:
 *   row_pairs:  corrections of the query rows' bigram pairs into the workspace;
 *   queries:    label scan of the query rows -> dsq, rowtau (uses row_pairs);
 *   keys:       label scan of the keys -> dsk, dv (length-1 part);
 *   key_pairs:  adds the keys' bigram-pair corrections to dsk, dv in place;
 *   tau_reduce: fixed-order reduction rowtau -> dtau. */
int32_t dism_hard_backward_row_pairs(const void* sq, const void* sk, const void* v,
                                     const void* dout, int32_t dtype, const int32_t* iq,
                                     const int32_t* ik, const uint8_t* hard,
                                     const int32_t* boundary, int32_t strip, const float* lut,
                                     const float* dlut, int64_t lut_stride, const float* lse2,
                                     int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                     void* workspace, int64_t workspace_bytes, void* stream);
int32_t dism_hard_backward_queries(const void* sq, const void* sk, const void* v,
                                   const void* dout, int32_t dtype, const int32_t* iq,
                                   const int32_t* ik, const uint8_t* hard,
                                   const int32_t* boundary, int32_t strip, const float* lut,
                                   const float* dlut, int64_t lut_stride, const float* lse2,
                                   int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                   void* workspace, int64_t workspace_bytes, float* dsq,
                                   float* rowtau, void* stream);
int32_t dism_hard_backward_keys(const void* sq, const void* sk, const void* v, const void* dout,
                                int32_t dtype, const int32_t* iq, const int32_t* ik,
                                const uint8_t* hard, const int32_t* boundary, int32_t strip,
                                const float* lut, int64_t lut_stride, const float* lse2,
                                int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                void* workspace, int64_t workspace_bytes, float* dsk, float* dv,
                                void* stream);
int32_t dism_hard_backward_key_pairs(const void* sq, const void* sk, const void* v,
                                     const void* dout, int32_t dtype, const int32_t* iq,
                                     const int32_t* ik, const uint8_t* hard,
                                     const int32_t* boundary, int32_t strip, const float* lut,
                                     int64_t lut_stride, const float* lse2, int64_t B, int64_t N,
                                     int64_t H, int32_t R, int32_t DV, void* workspace,
                                     int64_t workspace_bytes, float* dsk, float* dv,
                                     void* stream);
int32_t dism_hard_tau_reduce(const float* rowtau, int64_t B, int64_t H, int64_t N, float* dtau,
                             void* stream);

/* ---- Packed (varlen) batch-1 layouts.  One token sequence of N tokens (B = 1) holds the
 * documents [cu_seqlens[d], cu_seqlens[d+1]), d < docs (device int32 [docs+1], 0 = first,
 * N = last, non-decreasing: a repeated entry is an empty document, which is how a
 * fixed-capacity graph layout pads its table with entries equal to N); matches never cross a
 * document.  Hard flags are per training row: hard [rows, H] with N/rows tokens per row (a
 * multiple of 256), and no document crosses a training row (the caller checks the offsets on
 * the host, as the reference's layout does).  Soft training rows get zero outputs and
 * gradients.  Labels are any int32 values; 2 * N * docs <= 2^32 (documents are told apart by
 * tagging dense label ranks).  max_length is the longest document; the LUT covers lengths
 * 0..max_length.
 * Replaces the packed branches of cu.hard_readout / cu.hard_backward, which take the layout
 * table of dism_v3/python/flash_dism/varlen.py:9-51 (dism_v3/src/host/hard_forward.cpp:55-80,
 * dism_v3/src/host/hard_backward.cpp:54-93). */

/* Workspace bytes of a packed call (-1 for unsupported dimensions): the fixed-length
 * workspace of (1, N, H) plus the tagged labels and per-token document starts. */
int64_t dism_hard_packed_workspace_bytes(int64_t N, int64_t H, int32_t R, int32_t DV,
                                         int32_t dtype);

/* Ranks and tags the labels iq, ik [1,H,N] by document and prepares the workspace as
 * dism_hard_prepare does.  The readout and backward below read the labels from the
 * workspace. */
int32_t dism_hard_packed_prepare(const void* sq, const void* sk, const void* v, int32_t dtype,
                                 const int32_t* iq, const int32_t* ik,
                                 const int32_t* cu_seqlens, int64_t docs, int64_t N, int64_t H,
                                 int32_t R, int32_t DV, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/* Packed readout: O [1,N,H,DV], lse2 [1,H,N] (and optional lmax/jarg, key indices global),
 * equal per document to dism_hard_readout on that document alone.
 * Replaces cu.hard_readout with a layout table (dism_v3/src/host/hard_forward.cpp:55-80). */
int32_t dism_hard_packed_readout(const void* sq, const void* sk, const void* v, int32_t dtype,
                                 const uint8_t* hard, int64_t rows, const float* lut,
                                 int64_t lut_stride, int64_t max_length, int64_t N, int64_t H,
                                 int32_t R, int32_t DV, void* workspace, int64_t workspace_bytes,
                                 void* out, int32_t out_dtype, float* lse2, int32_t* lmax,
                                 int32_t* jarg, void* stream);

/* Packed backward (all five stages, then dtau over all hard documents).  The centring
 * constant of query i is G[i - start + 1] with the document-local position.
 * Replaces cu.hard_backward with a layout table (dism_v3/src/host/hard_backward.cpp:54-93). */
int32_t dism_hard_packed_backward(const void* sq, const void* sk, const void* v,
                                  const void* dout, int32_t dtype, const uint8_t* hard,
                                  int64_t rows, const float* lut, const float* dlut,
                                  int64_t lut_stride, int64_t max_length, const float* lse2,
                                  int64_t N, int64_t H, int32_t R, int32_t DV, void* workspace,
                                  int64_t workspace_bytes, float* dsq, float* dsk, float* dv,
                                  float* rowtau, float* dtau, void* stream);

/* ---- Inference (all rows hard, FP32 outputs).
 * Query resets follow the reference inference oracle (dism_v3/tests/test_sam_inference.py:9-29):
 * reset[b,h,i] = 1 starts query i's match afresh (its suffix walk stops at i); stored keys
 * stay visible. */

/* Workspace bytes of dism_hard_prefill (-1 for unsupported dimensions). */
int64_t dism_hard_prefill_workspace_bytes(int64_t B, int64_t N, int64_t H, int32_t R,
                                          int32_t DV, int32_t dtype);

/* Hard prefill: out [B,N,H,DV] fp32 and lse2 [B,H,N] for labels iq, ik [B,H,N] with optional
 * query resets [B,H,N] (uint8, NULL = none): prepare + readout of the training forward, every
 * row hard.  lut_stride >= N + 1.  The first n_valid positions of each row are the real tokens
 * (1 <= n_valid <= N; positions past it are padding that the dense-row classification does
 * not count).  Replaces HardDismPrefill's plan + execute
 * (dism_v3/python/flash_dism/inference/prefill_batch.py:67-118, README.md:229-292); equal
 * bit for bit to dism_hard_readout's fp32 output when there are no resets and no padding. */
int32_t dism_hard_prefill(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, const uint8_t* reset,
                          const float* lut, int64_t lut_stride, int64_t B, int64_t N,
                          int64_t n_valid, int64_t H, int32_t R, int32_t DV, void* workspace,
                          int64_t workspace_bytes, float* out, float* lse2, void* stream);

/* Incremental decoder state bytes for rows = B*H, capacity positions and `slots` label-table
 * entries per row (a power of two >= 64; at least twice the distinct key labels a row will
 * see), vectors cached in dtype (-1 for unsupported dimensions).  The first rows*4 int32 of
 * the state are, per row: position, list blocks used, last query reset, error flag (1 when
 * the label table overflowed).  No reference counterpart for the layout: the reference keeps
 * suffix-automaton snapshots (inference/runtime.py, gpu_runtime.py). */
int64_t dism_decoder_state_bytes(int64_t rows, int32_t R, int32_t DV, int64_t capacity,
                                 int32_t slots, int32_t dtype);

/* Zeroes a decoder state (a fill kernel on the stream). */
int32_t dism_decoder_init(void* state, int64_t state_bytes, int64_t rows, int32_t R, int32_t DV,
                          int64_t capacity, int32_t slots, int32_t dtype, void* stream);

/* Appends n tokens to every row: labels iq, ik [B,H,n], optional resets [B,H,n], vectors sq,
 * sk [B,n,H,R], v [B,n,H,DV] in the state's dtype.  Each token's key is added before its
 * query is read (a token matches itself).  out [B,n,H,DV] fp32 (and optional lse2 [B,H,n])
 * receive the outputs, equal bit for bit to the training forward's fp32 output at those
 * positions; out = NULL primes the state with keys only (sq and lut may then be NULL).
 * lut [H, lut_stride] with lut_stride >= capacity + 1.  The caller keeps position + n <=
 * capacity.  Replaces HardDismDecoder.append / prime
 * (dism_v3/python/flash_dism/inference/api.py:63-95). */
int32_t dism_decoder_step(void* state, int64_t state_bytes, int64_t B, int64_t H, int32_t R,
                          int32_t DV, int64_t capacity, int32_t slots, int32_t dtype, int64_t n,
                          const int32_t* iq, const int32_t* ik, const uint8_t* reset,
                          const void* sq, const void* sk, const void* v, const float* lut,
                          int64_t lut_stride, float* out, float* lse2, void* stream);

/* Workspace bytes of dism_decoder_prime for an n-token prompt (-1 for unsupported sizes). */
int64_t dism_decoder_prime_workspace_bytes(int64_t B, int64_t n, int64_t H, int32_t R,
                                           int32_t DV, int32_t dtype);

/* Primes a freshly initialised decoder state with an n-token prompt (keys only) in parallel:
 * the prompt's combined label order (dism_hard_prepare, rows padded to 256), then one wave per
 * (row, label bucket) builds each label's running matrix, count, last key and position list
 * with the same fp32 sequence as n single-token key steps, so decoding from it gives the
 * same outputs bit for bit.  Inputs as dism_decoder_step (no sq).  Replaces
 * HardDismDecoder.prime (dism_v3/python/flash_dism/inference/api.py:87-95). */
int32_t dism_decoder_prime(void* state, int64_t state_bytes, int64_t B, int64_t H, int32_t R,
                           int32_t DV, int64_t capacity, int32_t slots, int32_t dtype, int64_t n,
                           const int32_t* iq, const int32_t* ik, const uint8_t* reset,
                           const void* sk, const void* v, void* workspace,
                           int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DISM_HARD_H */
