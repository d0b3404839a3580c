// dism_aux.hip -- small kernels around the hard-core sweeps:
//   sign binarizer (labels), log2 weight table and its tau derivative, strip summaries,
//   summary composition (chunk pass), composed boundaries, deterministic tau reduction.
// All are HBM- or latency-bound elementwise/scan kernels; none of them is on the MFMA path.
#include "dism_device.h"
#include "dism_launch.h"

DISM_TU_LAYOUT(aux)

namespace dism {

// ---- labels: x [B,N,H,d] -> labels [B,H,N], bit k set iff x[...,k] > 0 (NaN, +-0 -> 0).
// Thread per (b,h,n) with n fastest so the int32 label stores are coalesced.
template <typename T>
__global__ __launch_bounds__(256) void sign_labels_kernel(const T* __restrict__ x, long B,
                                                          long N, long H, int d,
                                                          int32_t* __restrict__ out) {
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long total = B * H * N;
    if (t >= total) return;
    long n = t % N, bh = t / N, h = bh % H, b = bh / H;
    const T* row = x + ((b * N + n) * H + h) * d;
    int32_t lab = 0;
    if constexpr (sizeof(T) == 2) {
        if (d == 8 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {  // one 16-byte row
            const uint4 w = *reinterpret_cast<const uint4*>(row);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float v = (k & 1) ? __uint_as_float(ws[k >> 1] & 0xFFFF0000u)
                                        : __uint_as_float(ws[k >> 1] << 16);
                if (v > 0.0f) lab |= (1 << k);
            }
            out[t] = lab;
            return;
        }
    }
    for (int k = 0; k < d; ++k) {
        float v;
        if constexpr (sizeof(T) == 2) {
            v = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(row)[k] << 16);
        } else {
            v = reinterpret_cast<const float*>(row)[k];
        }
        if (v > 0.0f) lab |= (1 << k);
    }
    out[t] = lab;
}

// ---- weight tables: thread per (length, head)
__global__ __launch_bounds__(256) void log_weights_kernel(const float* __restrict__ tau,
                                                          long stride, float* __restrict__ out) {
    long l = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= stride) return;
    out[(long)blockIdx.y * stride + l] = log_weight(tau[blockIdx.y], l);
}

__global__ __launch_bounds__(256) void dlog_weights_kernel(const float* __restrict__ tau,
                                                           long stride, float* __restrict__ out) {
    long l = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= stride) return;
    out[(long)blockIdx.y * stride + l] = dlog_weight(tau[blockIdx.y], l);
}

// ---- strip summaries / composed boundaries.
// Entry (c, j) of a (b,h) row refers to the last row r = cS+S-1 of strip c.  One thread
// owns one signed diagonal d = r - j of one (b,h) and walks its strips in order, carrying
// the diagonal's running match length from strip to strip (the max-composition of the
// reference's chunk pass collapses to "add the previous strip's length when the whole strip
// segment matched").  Threads with d < 0 own only non-causal cells, which are -1.
//   composed = 1: j - L[r, j]               (hard_chunk_scan output)
//   composed = 0: last mismatching key coordinate inside the strip, -1 if none
//                 (summarize_hard output)
// fill_all = 0 skips the non-causal / soft-row -1 stores (the readout never reads them).
__global__ __launch_bounds__(256) void boundary_kernel(const int32_t* __restrict__ iq,
                                                       const int32_t* __restrict__ ik,
                                                       const uint8_t* __restrict__ hard,
                                                       int n, int strip, int composed,
                                                       int fill_all, int32_t* __restrict__ out) {
    int bh = blockIdx.y;
    int d = (int)((long)blockIdx.x * blockDim.x + threadIdx.x) - (n - 1);
    if (d > n - 1) return;
    long C = (n - 1) / strip;
    int32_t* o = out + (long)bh * C * n;
    const int32_t* q = iq + (long)bh * n;
    const int32_t* k = ik + (long)bh * n;
    bool on = hard[bh] != 0 && d >= 0;
    int carried = 0;
    for (long c = 0; c < C; ++c) {
        int r = (int)(c * strip + strip - 1);
        int j = r - d;
        if (j < 0 || j >= n) continue;
        if (!on) {
            if (fill_all) o[c * n + j] = -1;
            continue;
        }
        int cnt = 0;
        while (cnt < strip && j - cnt >= 0 && q[r - cnt] == k[j - cnt]) ++cnt;
        int value;
        if (composed) {
            int L = cnt == strip ? strip + carried : cnt;
            carried = L;
            value = j - L;
        } else {
            int seg = strip < j + 1 ? strip : j + 1;
            value = cnt == seg ? -1 : j - cnt;
        }
        o[c * n + j] = value;
    }
}

// ---- chunk pass over arbitrary strip-32 summaries (compose_cpu semantics):
//   out[c, j] = max(s[c, j], out[c-1, j-32]) for j >= 32, s[c, j] otherwise, then -1 for
//   non-causal j >= 32c+32.  Cells (c, j) -> (c+1, j+32) form independent chains; one thread
//   per chain.  Each chain reads an element before writing the same element, so in-place
//   use is safe.
__global__ __launch_bounds__(256) void chunk_kernel(const int32_t* __restrict__ summary,
                                                    int32_t* __restrict__ out, long C, int n) {
    long bh = blockIdx.y;
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    long chains = n + (C > 1 ? (C - 1) * 32 : 0);
    if (t >= chains) return;
    long c0, j0;
    if (t < n) { c0 = 0; j0 = t; } else { c0 = 1 + (t - n) / 32; j0 = (t - n) % 32; }
    const int32_t* s = summary + bh * C * n;
    int32_t* o = out + bh * C * n;
    int32_t prev = -1;
    for (long c = c0, j = j0; c < C && j < n; ++c, j += 32) {
        int32_t v = s[c * n + j];
        if (c > c0 && prev > v) v = prev;
        if (j >= c * 32 + 32) v = -1;
        o[c * n + j] = v;
        prev = v;
    }
}

// ---- tau reduction: dtau[h] = sum over (b, i) of rowtau[b,h,i], in the fixed order
// "blocks of TAU_BLOCK consecutive (b, i) rows summed sequentially in double, groups of
// TAU_GROUP consecutive block sums summed sequentially in double, then the group sums added
// sequentially in double", one workgroup per head.
constexpr int TAU_BLOCK = 64;
constexpr int TAU_GROUP = 32;
constexpr int TAU_THREADS = 1024;  // one block per lane: a round is TAU_THREADS / TAU_GROUP groups
static_assert(TAU_THREADS % TAU_GROUP == 0, "rounds hold whole groups");
// Each lane sums one block in order (16 float4 loads in flight when the block lies inside one
// aligned (b, h) row), lanes 0..31 sum one group each from LDS, lane 0 adds the round's group
// sums in order.  The chains are 64 + 32 + (groups) double adds long instead of one lane
// adding every block sum.
__global__ __launch_bounds__(TAU_THREADS) void tau_reduce_kernel(const float* __restrict__ rowtau,
                                                                 int B, int H, long n,
                                                                 float* __restrict__ dtau) {
    constexpr int GPR = TAU_THREADS / TAU_GROUP;  // groups per round
    __shared__ double part[TAU_THREADS];
    __shared__ double gsum[GPR];
    const int h = blockIdx.x, tid = threadIdx.x;
    const long total = (long)B * n;
    const long blocks = (total + TAU_BLOCK - 1) / TAU_BLOCK;
    const bool rows4 = n % TAU_BLOCK == 0 && (reinterpret_cast<uintptr_t>(rowtau) & 15) == 0;
    double outer = 0.0;
    for (long base = 0; base < blocks; base += TAU_THREADS) {
        const long blk = base + tid;
        double inner = 0.0;
        if (blk < blocks) {
            const long x0 = blk * TAU_BLOCK;
            if (rows4) {
                const long b = x0 / n, i = x0 - b * n;
                const float4* p = reinterpret_cast<const float4*>(rowtau + (b * H + h) * n + i);
                float4 w[TAU_BLOCK / 4];
#pragma unroll
                for (int u = 0; u < TAU_BLOCK / 4; ++u) w[u] = p[u];
#pragma unroll
                for (int u = 0; u < TAU_BLOCK / 4; ++u) {
                    inner += (double)w[u].x;
                    inner += (double)w[u].y;
                    inner += (double)w[u].z;
                    inner += (double)w[u].w;
                }
            } else {
                const long cnt = total - x0 < TAU_BLOCK ? total - x0 : TAU_BLOCK;
                for (long u = 0; u < cnt; ++u) {
                    const long x = x0 + u, b = x / n, i = x - b * n;
                    inner += (double)rowtau[(b * H + h) * n + i];
                }
            }
        }
        part[tid] = inner;
        __syncthreads();
        const long left = blocks - base;  // blocks of this round: min(left, TAU_THREADS)
        if (tid < GPR) {
            const long g0 = (long)tid * TAU_GROUP;
            const int cnt = left - g0 <= 0 ? 0 : (left - g0 < TAU_GROUP ? (int)(left - g0) : TAU_GROUP);
            double mid = 0.0;
            for (int u = 0; u < cnt; ++u) mid += part[g0 + u];
            gsum[tid] = mid;
        }
        __syncthreads();
        if (tid == 0) {
            const long gl = (left + TAU_GROUP - 1) / TAU_GROUP;
            const int ng = gl < GPR ? (int)gl : GPR;
            for (int u = 0; u < ng; ++u) outer += gsum[u];
        }
        __syncthreads();
    }
    if (tid == 0) dtau[h] = (float)outer;
}

// bf16 rows of d = 8 (16 bytes), H <= 64: a workgroup takes 64 positions x all H heads of one
// batch entry.  Loads run over (position, head) with the head fastest, one contiguous H*16-byte
// block per position; the labels go through LDS so that the stores run over positions, one
// contiguous 256-byte run per head.
constexpr int LAB_P = 64;
__global__ __launch_bounds__(256) void sign_labels_tile_kernel(const uint4* __restrict__ x,
                                                               long N, int H,
                                                               int32_t* __restrict__ out) {
    __shared__ int32_t s_lab[64][LAB_P + 1];
    const long tiles = (N + LAB_P - 1) / LAB_P;
    const long b = blockIdx.x / tiles, n0 = (blockIdx.x - b * tiles) * LAB_P;
    const int tid = threadIdx.x, cnt = LAB_P * H;
    for (int t = tid; t < cnt; t += 256) {
        const int nl = t / H, h = t - nl * H;
        int32_t lab = 0;
        if (n0 + nl < N) {
            const uint4 w = x[(b * N + n0 + nl) * H + h];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const float v = (k & 1) ? __uint_as_float(ws[k >> 1] & 0xFFFF0000u)
                                        : __uint_as_float(ws[k >> 1] << 16);
                if (v > 0.0f) lab |= (1 << k);
            }
        }
        s_lab[h][nl] = lab;
    }
    __syncthreads();
    for (int t = tid; t < cnt; t += 256) {
        const int h = t / LAB_P, nl = t - h * LAB_P;
        if (n0 + nl < N) out[(b * H + h) * N + n0 + nl] = s_lab[h][nl];
    }
}

// ---------------------------------------------------------------------------------------
hipError_t launch_sign_labels(const void* x, int dtype, long B, long N, long H, int d,
                              int32_t* out, hipStream_t s) {
    long total = B * H * N;
    if (dtype == DTYPE_BF16 && d == 8 && H <= 64 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        const long tiles = (N + LAB_P - 1) / LAB_P;
        hipLaunchKernelGGL(sign_labels_tile_kernel, dim3((unsigned)(B * tiles)), dim3(256), 0, s,
                           (const uint4*)x, N, (int)H, out);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((total + 255) / 256));
    if (dtype == DTYPE_BF16)
        hipLaunchKernelGGL(sign_labels_kernel<bf16_t>, grid, dim3(256), 0, s,
                           (const bf16_t*)x, B, N, H, d, out);
    else
        hipLaunchKernelGGL(sign_labels_kernel<float>, grid, dim3(256), 0, s, (const float*)x,
                           B, N, H, d, out);
    return hipGetLastError();
}

hipError_t launch_log_weights(const float* tau, int H, long stride, float* out, hipStream_t s) {
    dim3 grid((unsigned)((stride + 255) / 256), (unsigned)H);
    hipLaunchKernelGGL(log_weights_kernel, grid, dim3(256), 0, s, tau, stride, out);
    return hipGetLastError();
}

hipError_t launch_dlog_weights(const float* tau, int H, long stride, float* out, hipStream_t s) {
    dim3 grid((unsigned)((stride + 255) / 256), (unsigned)H);
    hipLaunchKernelGGL(dlog_weights_kernel, grid, dim3(256), 0, s, tau, stride, out);
    return hipGetLastError();
}

hipError_t launch_boundary(const int32_t* iq, const int32_t* ik, const uint8_t* hard, long BH,
                           int n, int strip, int composed, int fill_all, int32_t* out,
                           hipStream_t s) {
    dim3 grid((unsigned)((2L * n - 1 + 255) / 256), (unsigned)BH);
    hipLaunchKernelGGL(boundary_kernel, grid, dim3(256), 0, s, iq, ik, hard, n, strip,
                       composed, fill_all, out);
    return hipGetLastError();
}

hipError_t launch_chunk(const int32_t* summary, int32_t* out, long BH, long C, int n,
                        hipStream_t s) {
    long chains = n + (C > 1 ? (C - 1) * 32 : 0);
    dim3 grid((unsigned)((chains + 255) / 256), (unsigned)BH);
    hipLaunchKernelGGL(chunk_kernel, grid, dim3(256), 0, s, summary, out, C, n);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* p, long count, int32_t value) {
    long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e < count) p[e] = value;
}

hipError_t launch_fill_i32(int32_t* p, long count, int32_t value, hipStream_t s) {
    if (count <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, s, p,
                       count, value);
    return hipGetLastError();
}

hipError_t launch_tau_reduce(const float* rowtau, int B, int H, long n, float* dtau,
                             hipStream_t s) {
    hipLaunchKernelGGL(tau_reduce_kernel, dim3((unsigned)H), dim3(TAU_THREADS), 0, s, rowtau, B, H, n,
                       dtau);
    return hipGetLastError();
}

}  // namespace dism
