// dism_packed.hip -- packed batch-1 (varlen) layouts on the fixed-length kernels.
//
// A packed call holds documents [cu[d], cu[d+1]) of one sequence (B = 1; cu non-decreasing,
// a repeated entry is an empty document that no token belongs to, since a token's document is
// the LAST d with cu[d] <= t); matches never cross a document.  Instead of
// per-document task records the hard core runs unchanged on document-tagged labels:
//   tag = rank * docs + d   (uint32)
// with rank the dense rank of the raw label among the distinct labels of its (head) row --
// from the combined label order of the global-memory sort -- so tags are injective for any
// int32 labels and fit in 32 bits while 2N * docs <= 2^32.  A label group of the tagged row is
// one (label, document) group: the label scans reset at every document, and a bigram group
// only pairs positions of one document -- except the diagonal pair (p, p) at a document start
// p, whose predecessors (p-1, p-1) both lie in the previous document; the pair plan drops it.
// Suffix walks stop at the query's document start (dstart), and the backward's centring
// constant G[i+1] uses the document-local position.  Soft training rows are computed like hard
// ones (documents never cross a training row, so they never mix) and their outputs and
// gradients are zeroed afterwards.
#include "dism_device.h"
#include "dism_launch.h"

DISM_TU_LAYOUT(packed)

namespace dism {

// thread per token t: its document index and start; the first H tokens also write the
// all-ones row flags the kernels read (ones[h] = 1).
__global__ __launch_bounds__(256) void packed_docs_kernel(const int32_t* __restrict__ cu,
                                                          int docs, long H, long n,
                                                          int32_t* __restrict__ dstart,
                                                          int32_t* __restrict__ dindex,
                                                          uint8_t* __restrict__ ones) {
    const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n) return;
    int lo = 0, hi = docs;  // last document d with cu[d] <= t
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cu[mid] <= t) lo = mid; else hi = mid;
    }
    dstart[t] = cu[lo];
    dindex[t] = lo;
    for (long x = t; x < H; x += n) ones[x] = 1;
}

constexpr int TAG_THREADS = 1024, TAG_ITEMS = 8;

// block per (head) row: dense ranks from the sorted labels of the combined order (a label
// starts a new rank where it differs from its predecessor), then the tags at the entries'
// positions.  Chunks of TAG_THREADS * TAG_ITEMS entries, one block scan each.
__global__ __launch_bounds__(TAG_THREADS) void packed_tags_kernel(
    const int32_t* __restrict__ corder, const int32_t* __restrict__ clab,
    const int32_t* __restrict__ dindex, int docs, long n, int32_t* __restrict__ tq,
    int32_t* __restrict__ tk) {
    __shared__ int s_wave[TAG_THREADS / 64];
    __shared__ int s_carry;
    const long h = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const long n2 = 2 * n;
    const int32_t* lab = clab + h * n2;
    const int32_t* ord = corder + h * n2;
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (long base = 0; base < n2; base += (long)TAG_THREADS * TAG_ITEMS) {
        const long x0 = base + (long)tid * TAG_ITEMS;
        int head[TAG_ITEMS], c = 0;
        int prev = x0 > 0 && x0 <= n2 ? lab[x0 - 1] : 0;
#pragma unroll
        for (int u = 0; u < TAG_ITEMS; ++u) {
            const long x = x0 + u;
            const int cur = x < n2 ? lab[x] : prev;
            head[u] = x < n2 && (x == 0 || cur != prev);
            c += head[u];
            prev = cur;
        }
        // block exclusive scan of c
        int incl = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        if (lane == 63) s_wave[wave] = incl;
        __syncthreads();
        int before = s_carry;
        for (int w = 0; w < wave; ++w) before += s_wave[w];
        int r = before + incl - c;
#pragma unroll
        for (int u = 0; u < TAG_ITEMS; ++u) {
            const long x = x0 + u;
            if (x >= n2) break;
            r += head[u];
            const int ent = ord[x];
            const long p = ent >> 1;
            const uint32_t tag = (uint32_t)(r - 1) * (uint32_t)docs + (uint32_t)dindex[p];
            ((ent & 1) ? tq : tk)[h * n + p] = (int32_t)tag;
        }
        __syncthreads();
        if (tid == TAG_THREADS - 1) s_carry = before + incl;
        __syncthreads();
    }
}

// thread per (token t, head h), h fastest (BNHD rows are contiguous over h): zero every
// given output of tokens in soft training rows (hard[(t / row_tokens) * H + h] == 0).
__global__ __launch_bounds__(256) void packed_soft_zero_kernel(
    const uint8_t* __restrict__ hard, long row_tokens, long H, long n, int R, int DV,
    void* out, int out_dtype, float* lse2, int32_t* lmax, int32_t* jarg, float* dsq, float* dsk,
    float* dv, float* rowtau) {
    const long x = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= n * H) return;
    const long t = x / H, h = x - t * H;
    if (hard[(t / row_tokens) * H + h]) return;
    if (out) {
        if (out_dtype == DTYPE_F32)
            for (int d = 0; d < DV; ++d) reinterpret_cast<float*>(out)[x * DV + d] = 0.0f;
        else
            for (int d = 0; d < DV; ++d) reinterpret_cast<uint16_t*>(out)[x * DV + d] = 0;
    }
    const long bhn = h * n + t;
    if (lse2) lse2[bhn] = 0.0f;
    if (lmax) lmax[bhn] = 0;
    if (jarg) jarg[bhn] = -1;
    if (rowtau) rowtau[bhn] = 0.0f;
    if (dsq) for (int r = 0; r < R; ++r) dsq[x * R + r] = 0.0f;
    if (dsk) for (int r = 0; r < R; ++r) dsk[x * R + r] = 0.0f;
    if (dv) for (int d = 0; d < DV; ++d) dv[x * DV + d] = 0.0f;
}

hipError_t launch_packed_docs(const int32_t* cu, int docs, long H, long n, int32_t* dstart,
                              int32_t* dindex, uint8_t* ones, hipStream_t s) {
    hipLaunchKernelGGL(packed_docs_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       cu, docs, H, n, dstart, dindex, ones);
    return hipGetLastError();
}

hipError_t launch_packed_tags(const int32_t* corder, const int32_t* clab,
                              const int32_t* dindex, int docs, long H, long n, int32_t* tq,
                              int32_t* tk, hipStream_t s) {
    hipLaunchKernelGGL(packed_tags_kernel, dim3((unsigned)H), dim3(TAG_THREADS), 0, s, corder,
                       clab, dindex, docs, n, tq, tk);
    return hipGetLastError();
}

hipError_t launch_packed_soft_zero(const PackedZero& z, hipStream_t s) {
    const long total = z.n * z.H;
    hipLaunchKernelGGL(packed_soft_zero_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, s, z.hard, z.row_tokens, z.H, z.n, z.R, z.DV, z.out, z.out_dtype,
                       z.lse2, z.lmax, z.jarg, z.dsq, z.dsk, z.dv, z.rowtau);
    return hipGetLastError();
}

}  // namespace dism
