// dism_vocab.hip -- vocabulary (codebook) argmax labels: the general label producer.
//
// labels[b,h,t] = argmax_v  x[b,t,h,:] . vocab[h,v,:]   (first index wins on ties), the label
// rule of the reference (dism_v3/python/flash_dism/reference/dism_v3_ref.py:159-162, Triton
// emb_fwd dism_v3/python/flash_dism/emb_kernel.py:83-108; the softmax temperature beta > 0
// does not move the argmax).  The labels are those of EXACT arithmetic: every score is a sum
// of D products of bf16 values, each product exact in fp32.
//
// MI355X mapping: the scores are a [tokens x D] x [D x V] product, so the bulk goes to the
// matrix cores -- v_mfma_f32_32x32x8_bf16 tiles of 32 tokens x 32 vocabulary entries, one
// wave per 32-token tile of a (b,h) row, the tile's A fragments held in registers for the
// whole vocabulary.  Each lane keeps, per accumulator row, the best and second-best score of
// its vocabulary column class; a cross-lane merge gives per token (best, index, runner-up).
// fp32 accumulation of D exact products errs by at most D*2^-24*sum_d|x_d e_vd| <=
// D*2^-24*|x|_1*max|e| (eps below carries a 4x margin), so when best - runner-up > 2 eps the
// exact argmax is certain.  Otherwise (true ties, near ties) the wave rescores that token's
// whole vocabulary in fp64, summing d in order (exact for ordinary inputs; the CPU model
// sums in the same order), and takes the first maximal index.
#include "dism_path.h"

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
    int32_t* exact;        // optional counter of tokens rescored in fp64 (diagnostics)
};

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

template <int D>
__global__ __launch_bounds__(64 * VOC_WAVES) void vocab_argmax_kernel(VocabArgs a) {
    constexpr int KS = D / 8;  // 32x32x8 MFMA steps per tile
    __shared__ float s_sum_all[VOC_WAVES][32];
    __shared__ int s_amb_all[VOC_WAVES][32];
    float* s_sum = s_sum_all[wave_id()];
    int* s_amb = s_amb_all[wave_id()];
    const int lane = lane_id(), row = lane & 31, half = lane >> 5;
    const int tiles = (a.N + 31) / 32;
    const long item = (long)blockIdx.x * VOC_WAVES + wave_id();
    if (item >= (long)a.B * a.H * tiles) return;
    const int tile = (int)(item % tiles);
    const int bh = (int)(item / tiles), b = bh / a.H, h = bh % a.H;
    const int t0 = tile * 32;
    const int t = t0 + row;
    const bool tok = t < a.N;
    const bf16_t* xr = a.x + (((long)b * a.N + (tok ? t : 0)) * a.H + h) * D;
    const bf16_t* voc = a.vocab + (long)h * a.vhs;

    // A fragments: token row `row`, k = 8 ks + 4 half .. +3 (8 bytes); |x|_1 partials
    vshort4 af[KS];
    float l1 = 0.0f;
    bool sub = false;  // subnormal input: the matrix cores may flush it, so rescore exactly
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const uint2 w = tok ? *reinterpret_cast<const uint2*>(xr + ks * 8 + half * 4)
                            : make_uint2(0u, 0u);
        af[ks] = vshort4{(short)(w.x & 0xffff), (short)(w.x >> 16), (short)(w.y & 0xffff),
                         (short)(w.y >> 16)};
        l1 += fabsf(bf16_lo(w.x)) + fabsf(bf16_hi(w.x)) + fabsf(bf16_lo(w.y)) +
              fabsf(bf16_hi(w.y));
        sub = sub || subnormal2(w.x) || subnormal2(w.y);
    }
    l1 += __shfl_xor(l1, 32);
    sub = sub || __shfl_xor((int)sub, 32);
    // -1 marks a token with subnormal inputs (always rescored)
    if (half == 0) s_sum[row] = sub ? -1.0f : l1;

    // per accumulator j: rows (j/4)*8 + half*4 + j%4, column class `row` of each 32-tile
    float m1[16], m2[16];
    int i1[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        m1[j] = -INFINITY;
        m2[j] = -INFINITY;
        i1[j] = 0x7fffffff;
    }
    float emax = 0.0f;
    bool vsub = false;
    for (int v0 = 0; v0 < a.V; v0 += 32) {
        const int col = v0 + row;
        const bool vok = col < a.V;
        const bf16_t* vr = voc + (long)(vok ? col : 0) * D;
        vfloat16 c = {};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const uint2 w = vok ? *reinterpret_cast<const uint2*>(vr + ks * 8 + half * 4)
                                : make_uint2(0u, 0u);
            emax = fmaxf(emax, fmaxf(fmaxf(fabsf(bf16_lo(w.x)), fabsf(bf16_hi(w.x))),
                                     fmaxf(fabsf(bf16_lo(w.y)), fabsf(bf16_hi(w.y)))));
            vsub = vsub || subnormal2(w.x) || subnormal2(w.y);
            const vshort4 bf = {(short)(w.x & 0xffff), (short)(w.x >> 16),
                                (short)(w.y & 0xffff), (short)(w.y >> 16)};
            c = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(af[ks], bf, c, 0, 0, 0);
        }
        if (vok) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float s = c[j];
                if (s > m1[j]) {
                    m2[j] = m1[j];
                    m1[j] = s;
                    i1[j] = col;
                } else if (s > m2[j]) {
                    m2[j] = s;
                }
            }
        }
    }
    // merge over the 32 column classes (the lanes of each half)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) {
            const float o1 = __shfl_xor(m1[j], o), o2 = __shfl_xor(m2[j], o);
            const int oi = __shfl_xor(i1[j], o);
            merge_best(m1[j], i1[j], m2[j], o1, oi, o2);
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) emax = fmaxf(emax, __shfl_xor(emax, o));
    const bool any_vsub = __ballot(vsub) != 0ull;
    // s_sum (written by other lanes) is read below: keep the wave's LDS accesses in order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // decide: lanes 0 and 32 hold rows (j/4)*8 + half*4 + j%4
    if (row == 0) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = (j >> 2) * 8 + half * 4 + (j & 3);
            const int tt = t0 + r;
            if (tt >= a.N) continue;
            const float l1r = s_sum[r];
            const float eps = (float)(D + 4) * 0x1p-22f * l1r * emax + 0x1p-100f;
            const bool certain = !any_vsub && l1r >= 0.0f && m1[j] - m2[j] > 2.0f * eps;
            s_amb[r] = certain ? 0 : 1;
            if (certain) a.labels[(long)bh * a.N + tt] = i1[j];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // exact rescoring of the uncertain tokens, lanes over the vocabulary
    for (int r = 0; r < 32; ++r) {
        const int tt = t0 + r;
        if (tt >= a.N) break;
        if (!__builtin_amdgcn_readfirstlane(s_amb[r])) continue;
        const bf16_t* xt = a.x + (((long)b * a.N + tt) * a.H + h) * D;
        double best = -INFINITY;
        int bi = 0x7fffffff;
        for (int v = lane; v < a.V; v += 64) {
            const bf16_t* vr = voc + (long)v * D;
            double s = 0.0;
            for (int d = 0; d < D; ++d)
                s += (double)bf16f(reinterpret_cast<const uint16_t*>(xt)[d]) *
                     (double)bf16f(reinterpret_cast<const uint16_t*>(vr)[d]);
            if (s > best) {
                best = s;
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
        if (lane == 0) {
            a.labels[(long)bh * a.N + tt] = bi;
            if (a.exact) atomicAdd(a.exact, 1);
        }
    }
}

hipError_t launch_vocab_argmax(const void* x, const void* vocab, long vhs, int B, int N, int H,
                               int V, int D, int32_t* labels, int32_t* exact, hipStream_t s) {
    VocabArgs a{static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(vocab), vhs, B, N, H,
                V, labels, exact};
    const long items = (long)B * H * ((N + 31) / 32);
    const dim3 grid((unsigned)((items + VOC_WAVES - 1) / VOC_WAVES)), block(64 * VOC_WAVES);
    switch (D) {
        case 32: hipLaunchKernelGGL(vocab_argmax_kernel<32>, grid, block, 0, s, a); break;
        case 64: hipLaunchKernelGGL(vocab_argmax_kernel<64>, grid, block, 0, s, a); break;
        case 128: hipLaunchKernelGGL(vocab_argmax_kernel<128>, grid, block, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace dism
