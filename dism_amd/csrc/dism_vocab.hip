// dism_vocab.hip -- vocabulary (codebook) argmax labels: the general label producer.
//
// labels[b,h,t] = argmax_v  x[b,t,h,:] . vocab[h,v,:]   (first index wins on ties), the label
// rule of the reference (dism_v3/python/flash_dism/reference/dism_v3_ref.py:159-162, Triton
// emb_fwd dism_v3/python/flash_dism/emb_kernel.py:83-108; the softmax temperature beta > 0
// does not move the argmax).  The labels are those of EXACT arithmetic: every score is a sum
// of D products of bf16 values, each product exact in fp32.
//
// MI355X mapping: the scores are a [tokens x D] x [D x V] product, so the bulk goes to the
// matrix cores -- v_mfma_f32_32x32x8_bf16 tiles of 32 vocabulary rows (A) x 32 tokens (B),
// one wave per VOC_TT 32-token tiles of a (b,h) row with the token fragments held in
// registers for the whole vocabulary and the next vocabulary tile's fragments in flight.
// A lane holds one token's 16 scores of each tile and keeps a running (best, index,
// runner-up); the two half-waves merge at the end.
// fp32 accumulation of D exact products errs by at most D*2^-24*sum_d|x_d e_vd| <=
// D*2^-24*|x|_1*max|e| (eps below carries a 4x margin), so when best - runner-up > 2 eps the
// exact argmax is certain.  Otherwise (true ties, near ties) the wave rescores that token's
// whole vocabulary in fp64, summing d in order (exact for ordinary inputs; the CPU model
// sums in the same order), and takes the first maximal index.
#include "dism_path.h"

DISM_TU_LAYOUT(vocab)

namespace dism {

typedef short vshort4 __attribute__((ext_vector_type(4)));
typedef float vfloat16 __attribute__((ext_vector_type(16)));

constexpr int VOC_WAVES = 4;

struct VocabArgs {
    const bf16_t* x;       // [B,N,H,D]
    const bf16_t* vocab;   // [H,V,D] (head stride V*D) or shared [V,D] (head stride 0)
    long vhs;              // vocabulary head stride in elements
    int B, N, H, V;
    int32_t* labels;       // [B,H,N]
    int32_t* list;         // [1 + 2H + B*H*N]: count; per head max|e| (float bits) and a
                           // subnormal flag; then the (bh*N + t) of uncertain tokens
};

constexpr int VOC_STATS_THREADS = 256;

// per head: max |e| over the vocabulary and whether any entry is subnormal (the matrix cores
// may flush subnormals, so such a head is always rescored); block per head
__global__ __launch_bounds__(VOC_STATS_THREADS) void vocab_stats_kernel(VocabArgs a, int D) {
    __shared__ float s_m[VOC_STATS_THREADS / 64];
    __shared__ int s_f[VOC_STATS_THREADS / 64];
    const int h = blockIdx.x, tid = threadIdx.x;
    const uint32_t* w = reinterpret_cast<const uint32_t*>(a.vocab + (long)h * a.vhs);
    const long words = (long)a.V * D / 2;
    float m = 0.0f;
    bool sub = false;
    for (long i = tid; i < words; i += VOC_STATS_THREADS) {
        const uint32_t x = w[i];
        m = fmaxf(m, fmaxf(fabsf(bf16_lo(x)), fabsf(bf16_hi(x))));
        const uint32_t lo = x & 0x7fffu, hi = (x >> 16) & 0x7fffu;
        sub = sub || (lo != 0u && lo < 0x80u) || (hi != 0u && hi < 0x80u);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const bool any = __ballot(sub) != 0ull;
    if ((tid & 63) == 0) {
        s_m[tid >> 6] = m;
        s_f[tid >> 6] = any;
    }
    __syncthreads();
    if (tid == 0) {
        float mm = 0.0f;
        int ff = 0;
        for (int i = 0; i < VOC_STATS_THREADS / 64; ++i) {
            mm = fmaxf(mm, s_m[i]);
            ff |= s_f[i];
        }
        a.list[1 + 2 * h] = __float_as_int(mm);
        a.list[2 + 2 * h] = ff;
        if (h == 0) a.list[0] = 0;
    }
}

__device__ __forceinline__ float bf16f(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }

// either bf16 half of w is subnormal (zero exponent, nonzero mantissa)
__device__ __forceinline__ bool subnormal2(uint32_t w) {
    const uint32_t lo = w & 0x7fffu, hi = (w >> 16) & 0x7fffu;
    return (lo != 0u && lo < 0x80u) || (hi != 0u && hi < 0x80u);
}

// merge of (best, index, runner-up) summaries; equal bests keep the lower index and make the
// runner-up equal to the best (an exact tie is never certain)
__device__ __forceinline__ void merge_best(float& m1, int& i1, float& m2, float o1, int oi,
                                           float o2) {
    if (o1 > m1 || (o1 == m1 && oi < i1)) {
        m2 = fmaxf(m1, o2);
        m1 = o1;
        i1 = oi;
    } else {
        m2 = fmaxf(m2, o1);
    }
}

constexpr int VOC_TT = 2;  // 32-token tiles per wave (sharing every vocabulary fragment)

__device__ __forceinline__ vshort4 frag(uint2 w) {
    return vshort4{(short)(w.x & 0xffff), (short)(w.x >> 16), (short)(w.y & 0xffff),
                   (short)(w.y >> 16)};
}

// running (best, index, runner-up) of one accumulator register with score s at index col
__device__ __forceinline__ void take(float s, int col, float& m1, int& i1, float& m2) {
    const bool nb = s > m1;
    m2 = fmaxf(m2, nb ? m1 : s);
    i1 = nb ? col : i1;
    m1 = fmaxf(m1, s);
}

template <int D>
__global__ __launch_bounds__(64 * VOC_WAVES) void vocab_argmax_kernel(VocabArgs a) {
    constexpr int KS = D / 8;  // 32x32x8 MFMA steps per tile
    constexpr int TOK = 32 * VOC_TT;
    const int lane = lane_id(), row = lane & 31, half = lane >> 5;
    const int groups = (a.N + TOK - 1) / TOK;
    const long item = (long)blockIdx.x * VOC_WAVES + wave_id();
    if (item >= (long)a.B * a.H * groups) return;
    const int group = (int)(item % groups);
    const int bh = (int)(item / groups), b = bh / a.H, h = bh % a.H;
    const int t0 = group * TOK;
    const bf16_t* voc = a.vocab + (long)h * a.vhs;

    // token fragments (the B operand): token t0 + 32 u + row, k = 8 ks + 4 half .. +3; the
    // token's |x|_1 (both halves) and subnormal flag
    vshort4 tf[VOC_TT][KS];
    float l1[VOC_TT];
    bool sub[VOC_TT];
#pragma unroll
    for (int u = 0; u < VOC_TT; ++u) {
        const int t = t0 + 32 * u + row;
        const bool tok = t < a.N;
        const bf16_t* xr = a.x + (((long)b * a.N + (tok ? t : 0)) * a.H + h) * D + half * 4;
        float acc = 0.0f;
        bool sb = false;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint2 w = tok ? *reinterpret_cast<const uint2*>(xr + ks * 8) : make_uint2(0u, 0u);
            tf[u][ks] = frag(w);
            acc += fabsf(bf16_lo(w.x)) + fabsf(bf16_hi(w.x)) + fabsf(bf16_lo(w.y)) +
                   fabsf(bf16_hi(w.y));
            sb = sb || subnormal2(w.x) || subnormal2(w.y);
        }
        l1[u] = acc + __shfl_xor(acc, 32);
        sub[u] = sb || __shfl_xor((int)sb, 32);
    }

    // per token tile: the lane's running (best, index, runner-up) over the vocabulary rows it
    // holds -- rows v0 + (j/4)*8 + half*4 + j%4 of every 32-row tile, ascending
    float m1[VOC_TT], m2[VOC_TT];
    int i1[VOC_TT];
#pragma unroll
    for (int u = 0; u < VOC_TT; ++u) {
        m1[u] = -INFINITY;
        m2[u] = -INFINITY;
        i1[u] = 0x7fffffff;
    }
    auto load_a = [&](int v0, uint2 (&w)[KS]) {
        const int vr_i = v0 + row;
        const bool vok = vr_i < a.V;
        const bf16_t* vr = voc + (long)(vok ? vr_i : 0) * D + half * 4;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            w[ks] = vok ? *reinterpret_cast<const uint2*>(vr + ks * 8) : make_uint2(0u, 0u);
    };
    uint2 aw[KS], an[KS];
    load_a(0, aw);
    for (int v0 = 0; v0 < a.V; v0 += 32) {
        if (v0 + 32 < a.V) load_a(v0 + 32, an);  // next tile's fragments in flight
        vfloat16 c[VOC_TT];
#pragma unroll
        for (int u = 0; u < VOC_TT; ++u) c[u] = vfloat16{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const vshort4 vf = frag(aw[ks]);
#pragma unroll
            for (int u = 0; u < VOC_TT; ++u)
                c[u] = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(vf, tf[u][ks], c[u], 0, 0, 0);
        }
        if (v0 + 32 <= a.V) {
#pragma unroll
            for (int u = 0; u < VOC_TT; ++u)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    take(c[u][j], v0 + (j >> 2) * 8 + half * 4 + (j & 3), m1[u], i1[u], m2[u]);
        } else {
#pragma unroll
            for (int u = 0; u < VOC_TT; ++u)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int v = v0 + (j >> 2) * 8 + half * 4 + (j & 3);
                    if (v < a.V) take(c[u][j], v, m1[u], i1[u], m2[u]);
                }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) aw[ks] = an[ks];
    }
    const float emax = __int_as_float(a.list[1 + 2 * h]);
    const bool any_vsub = a.list[2 + 2 * h] != 0;
    // merge the two halves (same token, interleaved vocabulary rows); lanes < 32 decide and
    // list the uncertain tokens for the fp64 pass (one atomic per wave and tile)
#pragma unroll
    for (int u = 0; u < VOC_TT; ++u) {
        const float o1 = __shfl_xor(m1[u], 32), o2 = __shfl_xor(m2[u], 32);
        const int oi = __shfl_xor(i1[u], 32);
        merge_best(m1[u], i1[u], m2[u], o1, oi, o2);
        const int t = t0 + 32 * u + row;
        const float eps = (float)(D + 4) * 0x1p-22f * l1[u] * emax + 0x1p-100f;
        const bool certain = !any_vsub && !sub[u] && m1[u] - m2[u] > 2.0f * eps;
        const bool mine = half == 0 && t < a.N;
        if (mine && certain) a.labels[(long)bh * a.N + t] = i1[u];
        const unsigned long long m = __ballot(mine && !certain);
        if (m) {
            int base = 0;
            if (lane == 0) base = atomicAdd(a.list, __popcll(m));
            base = __shfl(base, 0);
            if (mine && !certain) {
                const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
                a.list[1 + 2 * a.H + base + __popcll(m & below)] = bh * a.N + t;
            }
        }
    }
}

// fp64 rescoring of the listed tokens: a persistent grid of waves strides over the list; a
// wave takes one token, the token row in LDS, lanes over the vocabulary, each score summed
// in d order in fp64 (the CPU model's order), first maximal index.
template <int D>
__global__ __launch_bounds__(64 * VOC_WAVES) void vocab_rescore_kernel(VocabArgs a) {
    __shared__ float s_x_all[VOC_WAVES][D];
    float* s_x = s_x_all[wave_id()];
    const int lane = lane_id();
    const int count = a.list[0];
    const int waves = (int)gridDim.x * VOC_WAVES;
    for (int e = (int)blockIdx.x * VOC_WAVES + wave_id(); e < count; e += waves) {
        const int id = a.list[1 + 2 * a.H + e];
        const int bh = id / a.N, t = id - bh * a.N, b = bh / a.H, h = bh % a.H;
        const bf16_t* voc = a.vocab + (long)h * a.vhs;
        const uint16_t* xt =
            reinterpret_cast<const uint16_t*>(a.x + (((long)b * a.N + t) * a.H + h) * D);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (int d = lane; d < D; d += 64) s_x[d] = bf16f(xt[d]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        double best = -INFINITY;
        int bi = 0x7fffffff;
        for (int v = lane; v < a.V; v += 64) {
            const uint4* vr = reinterpret_cast<const uint4*>(voc + (long)v * D);
            double sc = 0.0;
#pragma unroll 4
            for (int c8 = 0; c8 < D / 8; ++c8) {
                const uint4 w = vr[c8];
                const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    sc += (double)s_x[8 * c8 + 2 * k] * (double)bf16_lo(ws[k]);
                    sc += (double)s_x[8 * c8 + 2 * k + 1] * (double)bf16_hi(ws[k]);
                }
            }
            if (sc > best) {
                best = sc;
                bi = v;
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const double ob = __shfl_xor(best, o);
            const int oi = __shfl_xor(bi, o);
            if (ob > best || (ob == best && oi < bi)) {
                best = ob;
                bi = oi;
            }
        }
        if (lane == 0) a.labels[(long)bh * a.N + t] = bi;
    }
}

hipError_t launch_vocab_argmax(const void* x, const void* vocab, long vhs, int B, int N, int H,
                               int V, int D, int32_t* labels, int32_t* list, hipStream_t s) {
    VocabArgs a{static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(vocab), vhs, B, N, H,
                V, labels, list};
    hipLaunchKernelGGL(vocab_stats_kernel, dim3((unsigned)H), dim3(VOC_STATS_THREADS), 0, s, a,
                       D);
    const long items = (long)B * H * ((N + 32 * VOC_TT - 1) / (32 * VOC_TT));
    const dim3 grid((unsigned)((items + VOC_WAVES - 1) / VOC_WAVES)), block(64 * VOC_WAVES);
    const dim3 rgrid(256);  // persistent rescoring waves
    switch (D) {
        case 32:
            hipLaunchKernelGGL(vocab_argmax_kernel<32>, grid, block, 0, s, a);
            hipLaunchKernelGGL(vocab_rescore_kernel<32>, rgrid, block, 0, s, a);
            break;
        case 64:
            hipLaunchKernelGGL(vocab_argmax_kernel<64>, grid, block, 0, s, a);
            hipLaunchKernelGGL(vocab_rescore_kernel<64>, rgrid, block, 0, s, a);
            break;
        case 128:
            hipLaunchKernelGGL(vocab_argmax_kernel<128>, grid, block, 0, s, a);
            hipLaunchKernelGGL(vocab_rescore_kernel<128>, rgrid, block, 0, s, a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dism
