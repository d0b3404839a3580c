// dism_bucket.hip -- label buckets: stable counting sort of query and key positions by symbol.
//
// For every (batch, head) row and side (queries, keys) the positions are grouped by the symbol
// label & 255 and kept in ascending position order inside each bucket:
//   pos[bh][off[bh][s] .. off[bh][s+1])  = positions with symbol s, ascending
//   cs[bh][s] = sum_{s' < s} ceil(count(s') / 64)   (64-owner chunks before bucket s)
// The sweep kernels give one wave to each 64-owner chunk of a bucket and walk the opposite
// side's bucket of the same symbol, so every visited pair has equal low label bits; the full
// int32 labels are still compared, which keeps arbitrary int32 labels exact.
// Also: per-(batch, head) "contains a non-finite value" flags for value-like tensors, which
// select the masked accumulation path of the sweeps.
#include "dism_device.h"
#include "dism_launch.h"

namespace dism {

constexpr int BUCKET_THREADS = 1024;
constexpr int BUCKET_WAVES = BUCKET_THREADS / 64;

// grid (BH, 2): blockIdx.y = 0 queries, 1 keys
__global__ __launch_bounds__(BUCKET_THREADS) void bucket_kernel(BucketArgs a) {
    __shared__ int cnt[SYMBOLS];
    __shared__ int cursor[SYMBOLS];
    __shared__ int wcnt[BUCKET_WAVES][SYMBOLS];
    const int bh = blockIdx.x, side = blockIdx.y, n = a.n;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int32_t* __restrict__ lab = (side ? a.ik : a.iq) + (long)bh * n;
    int32_t* __restrict__ pos = (side ? a.kpos : a.qpos) + (long)bh * n;
    int32_t* __restrict__ off = (side ? a.koff : a.qoff) + (long)bh * (SYMBOLS + 1);
    int32_t* __restrict__ cs = (side ? a.kcs : a.qcs) + (long)bh * (SYMBOLS + 1);

    for (int s = tid; s < SYMBOLS; s += BUCKET_THREADS) cnt[s] = 0;
    __syncthreads();
    for (int x = tid; x < n; x += BUCKET_THREADS) atomicAdd(&cnt[lab[x] & (SYMBOLS - 1)], 1);
    __syncthreads();
    if (tid == 0) {  // 256-entry scans, sequential (negligible next to the scatter)
        int o = 0, c = 0;
        for (int s = 0; s < SYMBOLS; ++s) {
            off[s] = o;
            cs[s] = c;
            cursor[s] = o;
            o += cnt[s];
            c += (cnt[s] + 63) >> 6;
        }
        off[SYMBOLS] = o;
        cs[SYMBOLS] = c;
    }
    __syncthreads();
    const unsigned long long lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    for (int base = 0; base < n; base += BUCKET_THREADS) {
        const int x = base + tid;
        const bool ok = x < n;
        const int sym = ok ? (lab[x] & (SYMBOLS - 1)) : SYMBOLS;  // SYMBOLS = "no element"
        // lanes of this wave with the same symbol (9 ballots over the symbol bits)
        unsigned long long eq = ~0ull;
#pragma unroll
        for (int bit = 0; bit < 9; ++bit) {
            unsigned long long bal = __ballot((sym >> bit) & 1);
            eq &= ((sym >> bit) & 1) ? bal : ~bal;
        }
        const int rank = __popcll(eq & lt);
        for (int e = tid; e < BUCKET_WAVES * SYMBOLS; e += BUCKET_THREADS) (&wcnt[0][0])[e] = 0;
        __syncthreads();
        if (ok && rank == 0) wcnt[wave][sym] = __popcll(eq);
        __syncthreads();
        if (ok) {
            int before = cursor[sym];
            for (int w = 0; w < wave; ++w) before += wcnt[w][sym];
            pos[before + rank] = x;
        }
        __syncthreads();
        for (int s = tid; s < SYMBOLS; s += BUCKET_THREADS) {
            int add = 0;
            for (int w = 0; w < BUCKET_WAVES; ++w) add += wcnt[w][s];
            cursor[s] += add;
        }
        __syncthreads();
    }
}

// flags[bh] |= 1 if x[b, t, h, :] holds a non-finite value (x: [B,N,H,D], bf16 or f32)
template <typename T>
__global__ __launch_bounds__(256) void nonfinite_kernel(const T* __restrict__ x, long total,
                                                        int H, int D, long n, int32_t* flags) {
    long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    bool bad;
    if constexpr (sizeof(T) == 2) {
        uint32_t u = reinterpret_cast<const uint16_t*>(x)[e];
        bad = (u & 0x7F80u) == 0x7F80u;
    } else {
        uint32_t u = __float_as_uint(reinterpret_cast<const float*>(x)[e]);
        bad = (u & 0x7F800000u) == 0x7F800000u;
    }
    if (bad) {
        long row = e / D;                 // (b * n + t) * H + h
        long h = row % H, b = row / H / n;
        atomicOr(&flags[b * H + h], 1);
    }
}

// One thread per record.  Rows are copied with 16-byte vector accesses when the row length
// allows it; a record whose readout or value row holds a non-finite value raises bad[bh].
__device__ __forceinline__ bool word_nonfinite(uint32_t w, bool half) {
    if (half) return ((w & 0x7F80u) == 0x7F80u) || ((w & 0x7F800000u) == 0x7F800000u);
    return (w & 0x7F800000u) == 0x7F800000u;
}

__global__ __launch_bounds__(256) void records_kernel(RecordArgs a) {
    const long rec = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)a.B * a.H * a.n;
    if (rec >= total) return;
    const long bh = rec / a.n;
    const int p = a.pos[rec];
    const long b = bh / a.H, h = bh - b * a.H;
    const long row = (b * a.n + p) * a.H + h;
    const bool half = a.dtype == DTYPE_BF16;
    uint32_t* out = a.rec + rec * a.stride;
    const int32_t* lab = a.lab + bh * a.n;
    reinterpret_cast<uint4*>(out)[0] =
        make_uint4((uint32_t)p, (uint32_t)lab[p], p >= 1 ? (uint32_t)lab[p - 1] : 0u,
                   a.extra ? __float_as_uint(a.extra[bh * a.n + p]) : 0u);
    bool bad = false;
    const uint32_t* rr = reinterpret_cast<const uint32_t*>(a.rrow) + row * a.rw;
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(a.vrow) + row * a.vw;
    if ((a.rw & 3) == 0) {
        for (int c = 0; c < a.rw; c += 4) {
            uint4 x = *reinterpret_cast<const uint4*>(rr + c);
            bad |= word_nonfinite(x.x, half) | word_nonfinite(x.y, half) |
                   word_nonfinite(x.z, half) | word_nonfinite(x.w, half);
            *reinterpret_cast<uint4*>(out + 4 + c) = x;
        }
    } else {
        for (int c = 0; c < a.rw; ++c) {
            uint32_t x = rr[c];
            bad |= word_nonfinite(x, half);
            out[4 + c] = x;
        }
    }
    uint32_t* vo = out + 4 + a.rw;
    if ((a.rw & 3) == 0 && (a.vw & 3) == 0) {
        for (int c = 0; c < a.vw; c += 4) {
            uint4 x = *reinterpret_cast<const uint4*>(vr + c);
            bad |= word_nonfinite(x.x, half) | word_nonfinite(x.y, half) |
                   word_nonfinite(x.z, half) | word_nonfinite(x.w, half);
            *reinterpret_cast<uint4*>(vo + c) = x;
        }
    } else {
        for (int c = 0; c < a.vw; ++c) {
            uint32_t x = vr[c];
            bad |= word_nonfinite(x, half);
            vo[c] = x;
        }
    }
    if (bad) atomicOr(&a.bad[bh], 1);
}

hipError_t launch_records(const RecordArgs& a, hipStream_t s) {
    const long total = (long)a.B * a.H * a.n;
    hipLaunchKernelGGL(records_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_buckets(const BucketArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(bucket_kernel, dim3((unsigned)a.BH, 2), dim3(BUCKET_THREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_nonfinite(const void* x, int dtype, long B, long N, long H, int D,
                            int32_t* flags, hipStream_t s) {
    long total = B * N * H * D;
    dim3 grid((unsigned)((total + 255) / 256));
    if (dtype == DTYPE_BF16)
        hipLaunchKernelGGL(nonfinite_kernel<bf16_t>, grid, dim3(256), 0, s, (const bf16_t*)x,
                           total, (int)H, D, N, flags);
    else
        hipLaunchKernelGGL(nonfinite_kernel<float>, grid, dim3(256), 0, s, (const float*)x, total,
                           (int)H, D, N, flags);
    return hipGetLastError();
}

}  // namespace dism
