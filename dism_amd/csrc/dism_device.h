// dism_device.h -- device-side helpers shared by the flash_dism hard-core HIP kernels.
//
// Floating point contract: every kernel is compiled with -ffp-contract=off, fp32 division
// and sqrt correctly rounded, fp32 denormals preserved.  All multiply-adds that are meant to
// fuse are written as explicit fmaf/fma, so every kernel's result is a fixed sequence of IEEE
// operations that a CPU can repeat bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dism {

constexpr float LOG_ZERO = -1.0e6f;  // log2 weight of L=0 (reference LOG_ZERO)
constexpr int SYMBOLS = 256;          // prefilter alphabet: low 8 bits of the int32 label

struct bf16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// float -> bfloat16, round to nearest even, NaN kept quiet
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

// Load N consecutive elements of type T (bf16 or float) starting at p into fp32 registers.
// Rows are 16-byte aligned whenever N*sizeof(T) is a multiple of 16.
template <typename T, int N>
__device__ __forceinline__ void load_row(const T* p, float* out) {
    if constexpr (sizeof(T) == 2) {
        if constexpr (N % 2 == 1) {
            const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
            for (int c = 0; c < N; ++c) out[c] = __uint_as_float((uint32_t)q[c] << 16);
        } else if constexpr ((N * 2) % 16 == 0) {
            const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
            for (int c = 0; c < N / 8; ++c) {
                uint4 w = q[c];
                out[8 * c + 0] = bf16_lo(w.x); out[8 * c + 1] = bf16_hi(w.x);
                out[8 * c + 2] = bf16_lo(w.y); out[8 * c + 3] = bf16_hi(w.y);
                out[8 * c + 4] = bf16_lo(w.z); out[8 * c + 5] = bf16_hi(w.z);
                out[8 * c + 6] = bf16_lo(w.w); out[8 * c + 7] = bf16_hi(w.w);
            }
        } else if constexpr ((N * 2) % 8 == 0) {
            const uint2* q = reinterpret_cast<const uint2*>(p);
#pragma unroll
            for (int c = 0; c < N / 4; ++c) {
                uint2 w = q[c];
                out[4 * c + 0] = bf16_lo(w.x); out[4 * c + 1] = bf16_hi(w.x);
                out[4 * c + 2] = bf16_lo(w.y); out[4 * c + 3] = bf16_hi(w.y);
            }
        } else {
            const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
            for (int c = 0; c < N / 2; ++c) {
                uint32_t w = q[c];
                out[2 * c + 0] = bf16_lo(w); out[2 * c + 1] = bf16_hi(w);
            }
        }
    } else {
        if constexpr (N % 2 == 1) {
#pragma unroll
            for (int c = 0; c < N; ++c) out[c] = p[c];
        } else if constexpr ((N * 4) % 16 == 0) {
            const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
            for (int c = 0; c < N / 4; ++c) {
                float4 w = q[c];
                out[4 * c + 0] = w.x; out[4 * c + 1] = w.y; out[4 * c + 2] = w.z; out[4 * c + 3] = w.w;
            }
        } else {
            const float2* q = reinterpret_cast<const float2*>(p);
#pragma unroll
            for (int c = 0; c < N / 2; ++c) {
                float2 w = q[c];
                out[2 * c + 0] = w.x; out[2 * c + 1] = w.y;
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// exp2 / log2 in fp32, written from the mathematics (Cody-Waite style reduction + fitted
// polynomial); identical operation sequence to the CPU model.
// exp2: x = n + f, n = rint(x), |f| <= 1/2; 2^f by a degree-6 polynomial fitted for this
// project (max relative error 1.3 ulp including rounding); 2^n through the exponent field.
__device__ __forceinline__ float exp2_fp32(float x) {
    if (x != x) return x;
    if (!(x >= -149.0f)) return 0.0f;
    if (x >= 128.0f) return __uint_as_float(0x7F800000u);
    float n = __builtin_rintf(x);
    float f = x - n;
    float p = 0x1.41d3e2p-13f;
    p = __builtin_fmaf(p, f, 0x1.5f456cp-10f);
    p = __builtin_fmaf(p, f, 0x1.3b2dbap-7f);
    p = __builtin_fmaf(p, f, 0x1.c6aed4p-5f);
    p = __builtin_fmaf(p, f, 0x1.ebfbdap-3f);
    p = __builtin_fmaf(p, f, 0x1.62e430p-1f);
    p = __builtin_fmaf(p, f, 0x1.000000p+0f);
    int ni = (int)n;
    if (ni > 127) { p = p * 2.0f; ni -= 1; }
    if (ni < -126) { p = p * 0x1p-64f; ni += 64; }
    return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

// log2 of a positive normal float: x = m 2^e with m in [sqrt(1/2), sqrt(2)),
// s = (m-1)/(m+1), log2 m = s * sum_k 2/((2k+1) ln 2) s^(2k) (six terms).
__device__ __forceinline__ float log2_fp32(float x) {
    uint32_t b = __float_as_uint(x);
    int e = (int)((b >> 23) & 255u) - 127;
    float m = __uint_as_float((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 0x1.6a09e6p+0f) { m = m * 0.5f; e += 1; }
    float s = (m - 1.0f) / (m + 1.0f);
    float t = s * s;
    float p = 0x1.0c9a84p-2f;
    p = __builtin_fmaf(p, t, 0x1.484b14p-2f);
    p = __builtin_fmaf(p, t, 0x1.a61762p-2f);
    p = __builtin_fmaf(p, t, 0x1.2776c6p-1f);
    p = __builtin_fmaf(p, t, 0x1.ec709ep-1f);
    p = __builtin_fmaf(p, t, 0x1.715476p+1f);
    return (float)e + s * p;
}

// ---------------------------------------------------------------------------------------
// Double-precision helpers for the per-head weight tables (H x (N+1) entries per call, so
// fp64 VALU cost is irrelevant).  Only IEEE basic operations and fma are used.
constexpr double LN2 = 0x1.62e42fefa39efp-1;
constexpr double LN2_HI = 0x1.62e42fee00000p-1;
constexpr double LN2_LO = 0x1.a39ef35793c76p-33;
constexpr double INV_LN2 = 0x1.71547652b82fep+0;

__device__ __forceinline__ double inv_fact(int k) {
    constexpr double T[19] = {
        1.0, 1.0, 1.0 / 2.0, 1.0 / 6.0, 1.0 / 24.0, 1.0 / 120.0, 1.0 / 720.0, 1.0 / 5040.0,
        1.0 / 40320.0, 1.0 / 362880.0, 1.0 / 3628800.0, 1.0 / 39916800.0, 1.0 / 479001600.0,
        1.0 / 6227020800.0, 1.0 / 87178291200.0, 1.0 / 1307674368000.0,
        1.0 / 20922789888000.0, 1.0 / 355687428096000.0, 1.0 / 6402373705728000.0};
    return T[k];
}

// natural log of a positive normal double: atanh series in s = (m-1)/(m+1), 14 terms
__device__ __forceinline__ double log_fp64(double x) {
    uint64_t b = (uint64_t)__double_as_longlong(x);
    int e = (int)((b >> 52) & 0x7FFu) - 1023;
    double m = __longlong_as_double((long long)((b & 0xFFFFFFFFFFFFFull) | 0x3FF0000000000000ull));
    if (m > 0x1.6a09e667f3bcdp+0) { m = m * 0.5; e += 1; }
    double s = (m - 1.0) / (m + 1.0);
    double t = s * s;
    double p = 1.0 / 27.0;
    for (int k = 12; k >= 0; --k) p = __builtin_fma(p, t, 1.0 / (double)(2 * k + 1));
    return __builtin_fma((double)e, LN2, (2.0 * s) * p);
}

// e^x: n = rint(x / ln2), r = x - n ln2 in two parts, Taylor polynomial of degree 16
__device__ __forceinline__ double exp_fp64(double x) {
    if (x < -745.0) return 0.0;
    if (x > 709.0) return __longlong_as_double(0x7FF0000000000000ll);
    double n = __builtin_rint(x * INV_LN2);
    double r = __builtin_fma(-n, LN2_HI, x);
    r = __builtin_fma(-n, LN2_LO, r);
    double p = inv_fact(16);
    for (int k = 15; k >= 0; --k) p = __builtin_fma(p, r, inv_fact(k));
    int ni = (int)n;
    if (ni < -1022) { p = p * 0x1p-60; ni += 60; }
    return p * __longlong_as_double((long long)((uint64_t)(ni + 1023) << 52));
}

// q(x) = (1 - e^-x) / x for x >= 0, q(0) = 1
__device__ __forceinline__ double one_minus_exp_neg_over(double x) {
    if (x < 1.0) {
        double p = inv_fact(18);
        for (int k = 17; k >= 1; --k) p = __builtin_fma(p, -x, inv_fact(k));
        return p;
    }
    return (1.0 - exp_fp64(-x)) / x;
}

// e^x - 1 for x >= 0
__device__ __forceinline__ double expm1_fp64(double x) {
    if (x < 1.0) {
        double p = inv_fact(18);
        for (int k = 17; k >= 1; --k) p = __builtin_fma(p, x, inv_fact(k));
        return x * p;
    }
    return exp_fp64(x) - 1.0;
}

// log2 W_L with W_L = sum_{s=1..L} e^{s tau}:
//   ln W_L = (tau > 0 ? L tau : tau) + ln L + ln q(L |tau|) - ln q(|tau|)
// (the geometric sum factored around its largest term; no cancellation near tau = 0).
__device__ __forceinline__ float log_weight(float tau, long L) {
    if (L <= 0) return LOG_ZERO;
    double t = (double)tau, a = t < 0.0 ? -t : t, l = (double)L;
    double lead = t > 0.0 ? l * t : t;
    double r = lead + log_fp64(l);
    r = r + log_fp64(one_minus_exp_neg_over(l * a));
    r = r - log_fp64(one_minus_exp_neg_over(a));
    return (float)(r * INV_LN2);
}

// g_L = d ln W_L / d tau.  For |L tau| < 0.1 the series of
// g = (L+1)/2 + (L coth(L tau/2) - coth(tau/2))/2; otherwise the closed form
// tau > 0: L + L/expm1(L a) - 1/expm1(a);  tau < 0: 1 - L/expm1(L a) + 1/expm1(a).
__device__ __forceinline__ float dlog_weight(float tau, long L) {
    if (L <= 0) return 0.0f;
    double t = (double)tau, l = (double)L, x = l * t;
    double ax = x < 0.0 ? -x : x;
    if (ax < 0.1) {
        const double C[6] = {1.0 / 12.0, -1.0 / 720.0, 1.0 / 30240.0, -1.0 / 1209600.0,
                             1.0 / 47900160.0, -691.0 / 1307674368000.0};
        double l2 = l * l, t2 = t * t, lp = l2;
        double terms[6];
        for (int n = 0; n < 6; ++n) { terms[n] = C[n] * (lp - 1.0); lp = lp * l2; }
        double acc = terms[5];
        for (int n = 4; n >= 0; --n) acc = __builtin_fma(acc, t2, terms[n]);
        return (float)__builtin_fma(t, acc, (l + 1.0) * 0.5);
    }
    double a = t < 0.0 ? -t : t;
    double big = l / expm1_fp64(l * a);
    double small = 1.0 / expm1_fp64(a);
    double g = t > 0.0 ? (l + big) - small : (1.0 - big) + small;
    return (float)g;
}

// ---------------------------------------------------------------------------------------
// Match length at a verified match (i, j) of one (batch, head) row: walk up-left along the
// diagonal.  With a composed boundary table of strip height S (row c holds, for the last
// row r = cS+S-1 of strip c, the last mismatching key coordinate j - L[r, j]), the walk
// never leaves the current strip; without one it walks to the first mismatch.
__device__ __forceinline__ int match_length(const int32_t* __restrict__ q,
                                            const int32_t* __restrict__ k, int i, int j,
                                            const int32_t* __restrict__ bound, int strip,
                                            int n) {
    int lo = bound ? (i / strip) * strip : 0;
    int c = 1;
    while (i - c >= lo && j - c >= 0 && q[i - c] == k[j - c]) ++c;
    if (bound && lo > 0 && i - c < lo && j - c >= 0) {
        int jj = j - c;
        c += jj - bound[(long)(lo / strip - 1) * n + jj];
    }
    return c;
}

}  // namespace dism
