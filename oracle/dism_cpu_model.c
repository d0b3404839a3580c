/*
 * dism_cpu_model.c -- CPU restatement of the flash_dism hard (integer-label) core.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker and the timed CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product path (dism_amd/) never calls into it.
 *
 * What it restates (reference paths relative to /root/reference):
 *   - match length recurrence L[i,j] = (iq[i]==ik[j]) ? L[i-1,j-1]+1 : 0, computed here
 *     with the textbook two-row dynamic programme (dism_v3/tests/test_hard_chunk.py:24-36,
 *     dense_boundary), NOT with the GPU's walk-back + boundary method;
 *   - strip summaries R (dism_v3/tests/test_hard_summary.py:37-49) and their max
 *     composition (dism_v3/tests/test_hard_chunk.py:14-21, compose_cpu);
 *   - log2 geometric-weight table (dism_v3/src/hard_forward.cu:10-25) and its natural-tau
 *     derivative (dism_v3/src/hard_backward.cu:8-23);
 *   - normalised signed readout with online max starting at 0 and unit fallback
 *     (dism_v3/include/forward/readout.cuh:16-61, store_output :63-100);
 *   - explicit backward dSQ/dSK/dV and the centred four-moment dtau
 *     (dism_v3/python/flash_dism/reference/dism_v3_ref.py:108-127,
 *      dism_v3/src/hard_backward.cu:71-120,156-197).
 *
 * Floating point: the fp32 operation sequence per query row / per key is the one the
 * HIP kernels document (ascending key order per row, ascending query order per key,
 * explicit fmaf, software exp2/log2 from the same published method), so outputs can be
 * compared bit for bit.  Build with -ffp-contract=off.  The LUT/dLUT are evaluated in
 * double with series/Horner schemes using only IEEE basic operations.
 *
 * Parity pinning of each function is listed in tests/test_oracle.py.
 */
#define _GNU_SOURCE
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LOG_ZERO (-1.0e6f)

static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

/* ---------------- fp32 exp2 / log2 (Cody-Waite reduction + polynomial) -------------
 * exp2: x = n + f, n = rint(x), |f| <= 1/2, 2^f by a degree-6 least-squares minimax
 * polynomial (coefficients fitted for this project, max rel err 1.3 ulp incl. rounding),
 * scaled by 2^n through the exponent field. */
static const float E2C[7] = {0x1.000000p+0f, 0x1.62e430p-1f, 0x1.ebfbdap-3f, 0x1.c6aed4p-5f,
                             0x1.3b2dbap-7f, 0x1.5f456cp-10f, 0x1.41d3e2p-13f};

float orc_exp2f(float x) {
    if (x != x) return x;
    if (!(x >= -149.0f)) return 0.0f;
    if (x >= 128.0f) return INFINITY;
    float n = rintf(x);
    float f = x - n;
    float p = E2C[6];
    for (int k = 5; k >= 0; --k) p = fmaf(p, f, E2C[k]);
    int ni = (int)n;
    if (ni > 127) { p = p * 2.0f; ni -= 1; }
    if (ni < -126) { p = p * 0x1p-64f; ni += 64; }
    return p * u2f((uint32_t)(ni + 127) << 23);
}

/* log2 of a positive normal float: x = m 2^e, m in [sqrt(1/2), sqrt(2)), s=(m-1)/(m+1),
 * log2 m = s * sum_k 2/((2k+1) ln 2) s^(2k), six terms. */
static const float L2C[6] = {0x1.715476p+1f, 0x1.ec709ep-1f, 0x1.2776c6p-1f,
                             0x1.a61762p-2f, 0x1.484b14p-2f, 0x1.0c9a84p-2f};

float orc_log2f(float x) {
    uint32_t b = f2u(x);
    int e = (int)((b >> 23) & 255u) - 127;
    float m = u2f((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 0x1.6a09e6p+0f) { m = m * 0.5f; e += 1; }
    float s = (m - 1.0f) / (m + 1.0f);
    float t = s * s;
    float p = L2C[5];
    for (int k = 4; k >= 0; --k) p = fmaf(p, t, L2C[k]);
    return (float)e + s * p;
}

/* ---------------- double helpers for the weight tables ---------------- */
static const double LN2 = 0x1.62e42fefa39efp-1;
static const double LN2_HI = 0x1.62e42fee00000p-1;
static const double LN2_LO = 0x1.a39ef35793c76p-33;
static const double INV_LN2 = 0x1.71547652b82fep+0;

/* natural log, x > 0 normal: atanh series in s=(m-1)/(m+1), 14 terms */
double orc_logd(double x) {
    uint64_t b = d2u(x);
    int e = (int)((b >> 52) & 0x7ffu) - 1023;
    double m = u2d((b & 0xFFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
    if (m > 0x1.6a09e667f3bcdp+0) { m = m * 0.5; e += 1; }
    double s = (m - 1.0) / (m + 1.0);
    double t = s * s;
    double p = 1.0 / 27.0;
    for (int k = 12; k >= 0; --k) p = fma(p, t, 1.0 / (double)(2 * k + 1));
    return fma((double)e, LN2, (2.0 * s) * p);
}

static const double INV_FACT[19] = {
    1.0, 1.0, 1.0 / 2.0, 1.0 / 6.0, 1.0 / 24.0, 1.0 / 120.0, 1.0 / 720.0, 1.0 / 5040.0,
    1.0 / 40320.0, 1.0 / 362880.0, 1.0 / 3628800.0, 1.0 / 39916800.0, 1.0 / 479001600.0,
    1.0 / 6227020800.0, 1.0 / 87178291200.0, 1.0 / 1307674368000.0, 1.0 / 20922789888000.0,
    1.0 / 355687428096000.0, 1.0 / 6402373705728000.0};

/* e^x for x <= 709: n = rint(x/ln2), r = x - n ln2 (two-part), Taylor degree 16 */
double orc_expd(double x) {
    if (x < -745.0) return 0.0;
    if (x > 709.0) return INFINITY;
    double n = rint(x * INV_LN2);
    double r = fma(-n, LN2_HI, x);
    r = fma(-n, LN2_LO, r);
    double p = INV_FACT[16];
    for (int k = 15; k >= 0; --k) p = fma(p, r, INV_FACT[k]);
    int ni = (int)n;
    if (ni < -1022) { p = p * 0x1p-60; ni += 60; }
    return p * u2d((uint64_t)(ni + 1023) << 52);
}

/* (1 - e^-x)/x for x >= 0 (equals 1 at 0) */
double orc_one_minus_exp_neg_over(double x) {
    if (x < 1.0) {
        double p = INV_FACT[18];
        for (int k = 17; k >= 1; --k) p = fma(p, -x, INV_FACT[k]);
        return p;
    }
    return (1.0 - orc_expd(-x)) / x;
}

/* e^x - 1 for x >= 0 */
double orc_expm1d(double x) {
    if (x < 1.0) {
        double p = INV_FACT[18];
        for (int k = 17; k >= 1; --k) p = fma(p, x, INV_FACT[k]);
        return x * p;
    }
    return orc_expd(x) - 1.0;
}

/* log2 W_L, W_L = sum_{s=1..L} e^{s tau}; W_0 -> LOG_ZERO.
 * log W = (tau>0 ? L tau : tau) + ln L + ln q(L|tau|) - ln q(|tau|), q(x)=(1-e^-x)/x.
 * Reference branches: dism_v3/src/hard_forward.cu:15-22. */
float orc_log_weight(float tau, long L) {
    if (L <= 0) return LOG_ZERO;
    double t = (double)tau, a = fabs(t), l = (double)L;
    double lead = t > 0.0 ? l * t : t;
    double r = lead + orc_logd(l);
    r = r + orc_logd(orc_one_minus_exp_neg_over(l * a));
    r = r - orc_logd(orc_one_minus_exp_neg_over(a));
    return (float)(r * INV_LN2);
}

/* g_L = d ln W_L / d tau (natural units).  Series for |L tau| < 0.1 from
 * g = (L+1)/2 + (L coth(L tau/2) - coth(tau/2))/2, closed form elsewhere.
 * Reference: dism_v3/src/hard_backward.cu:8-23. */
float orc_dlog_weight(float tau, long L) {
    if (L <= 0) return 0.0f;
    double t = (double)tau, l = (double)L, x = l * t;
    if (fabs(x) < 0.1) {
        static const double C[6] = {1.0 / 12.0, -1.0 / 720.0, 1.0 / 30240.0, -1.0 / 1209600.0,
                                    1.0 / 47900160.0, -691.0 / 1307674368000.0};
        double l2 = l * l, t2 = t * t;
        double lp = l2, acc;
        double terms[6];
        for (int n = 0; n < 6; ++n) { terms[n] = C[n] * (lp - 1.0); lp = lp * l2; }
        acc = terms[5];
        for (int n = 4; n >= 0; --n) acc = fma(acc, t2, terms[n]);
        return (float)(fma(t, acc, (l + 1.0) * 0.5));
    }
    double a = fabs(t);
    double big = l / orc_expm1d(l * a);
    double small = 1.0 / orc_expm1d(a);
    double g = t > 0.0 ? (l + big) - small : (1.0 - big) + small;
    return (float)g;
}

void orc_lut(const float* tau, int heads, long stride, float* out) {
    for (int h = 0; h < heads; ++h)
        for (long l = 0; l < stride; ++l) out[(long)h * stride + l] = orc_log_weight(tau[h], l);
}

void orc_dlut(const float* tau, int heads, long stride, float* out) {
    for (int h = 0; h < heads; ++h)
        for (long l = 0; l < stride; ++l) out[(long)h * stride + l] = orc_dlog_weight(tau[h], l);
}

/* ---------------- integer core ---------------- */

/* Sign binarizer: label = sum_d [x_d > 0] 2^d (x [rows, d], labels [rows]) */
void orc_sign_labels(const float* x, long rows, int d, int32_t* out) {
    for (long r = 0; r < rows; ++r) {
        int32_t lab = 0;
        for (int k = 0; k < d; ++k)
            if (x[r * d + k] > 0.0f) lab |= (1 << k);
        out[r] = lab;
    }
}

/* Strip summaries (composed=0) or composed boundaries (composed=1), strip height S.
 * out [B,H,(N-1)/S,N]; entry (c,j): row r=cS+S-1; causal j<=r on hard rows; else -1.
 * composed: j - L[r,j] with L the full-history match length (dense_boundary).
 * summary : last mismatching key coordinate inside strip c, -1 if none (oracle :37-49). */
void orc_boundary(const int32_t* iq, const int32_t* ik, const uint8_t* hard, int B, int H,
                  long N, int S, int composed, int32_t* out) {
    long C = (N - 1) / S;
    int32_t* len = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
    int32_t* prv = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
    for (int bh = 0; bh < B * H; ++bh) {
        const int32_t* q = iq + (long)bh * N;
        const int32_t* k = ik + (long)bh * N;
        int32_t* o = out + (long)bh * C * N;
        for (long x = 0; x < C * N; ++x) o[x] = -1;
        if (!hard[bh]) continue;
        if (composed) {
            for (long j = 0; j < N; ++j) len[j] = 0;
            for (long row = 0; row < C * S; ++row) {
                for (long j = N - 1; j >= 0; --j) {
                    int32_t in = j ? len[j - 1] : 0;
                    len[j] = (q[row] == k[j]) ? in + 1 : 0;
                }
                if (row % S == S - 1) {
                    long c = row / S;
                    for (long j = 0; j <= row && j < N; ++j) o[c * N + j] = (int32_t)(j - len[j]);
                }
            }
        } else {
            for (long c = 0; c < C; ++c) {
                for (long j = 0; j < N; ++j) prv[j] = -1;
                for (long row = c * S; row < c * S + S; ++row) {
                    for (long j = N - 1; j >= 0; --j) {
                        int32_t in = j ? prv[j - 1] : -1;
                        int32_t here = (q[row] == k[j]) ? -1 : (int32_t)j;
                        prv[j] = in > here ? in : here;
                    }
                }
                for (long j = 0; j <= c * S + S - 1 && j < N; ++j) o[c * N + j] = prv[j];
            }
        }
    }
    free(len);
    free(prv);
}

/* compose_cpu (test_hard_chunk.py:14-21): summaries [BH,C,N], strip 32 */
void orc_chunk(const int32_t* summary, long BH, long C, long N, int32_t* out) {
    memcpy(out, summary, sizeof(int32_t) * (size_t)(BH * C * N));
    for (long bh = 0; bh < BH; ++bh) {
        int32_t* r = out + bh * C * N;
        for (long c = 0; c < C; ++c) {
            if (c)
                for (long j = 32; j < N; ++j) {
                    int32_t a = r[c * N + j], b = r[(c - 1) * N + j - 32];
                    r[c * N + j] = a > b ? a : b;
                }
            for (long j = c * 32 + 32; j < N; ++j) r[c * N + j] = -1;
        }
    }
}

/* Brute-force match length at (i,j) by direct suffix walk (tiny-input pin). */
long orc_suffix_walk(const int32_t* q, const int32_t* k, long i, long j) {
    long c = 0;
    while (i - c >= 0 && j - c >= 0 && q[i - c] == k[j - c]) ++c;
    return c;
}

/* The walk of a query whose match was reset at position lo <= i (the reference inference
 * oracle masks the predecessor score of a reset query, test_sam_inference.py:19-21): the
 * query side never reaches below lo. */
long orc_suffix_walk_from(const int32_t* q, const int32_t* k, long i, long j, long lo) {
    long c = 0;
    while (i - c >= lo && j - c >= 0 && q[i - c] == k[j - c]) ++c;
    return c;
}

/* ---------------- direct (pairwise) definition ----------------
 * Vectors fp32 BNHD (bf16 inputs widened exactly by the caller), labels BHN, hard [B*H].
 * Match lengths come from the two-row dynamic programme L[i,j] = (q[i]==k[j]) ?
 * L[i-1,j-1]+1 : 0, with L[i-1,*] taken as 0 at a query reset (i == wlo[i]).
 * Forward, per query row i:
 *   pass 1 (integer): L for every matching key; m = max(0, max_j LUT[L]); longest match with
 *                     ties -> largest j;
 *   pass 2, ascending j over matches:
 *     den starts at exp2(-m); p = exp2(LUT[L] - m); den += p;
 *     s = fma-chain(sq_i . sk_j); ps = p*s; acc = fma(ps, v_j, acc)
 *   out = acc/den, lse2 = m + log2(den).
 * This is the reference's online-max readout (readout.cuh:16-61) with the final maximum
 * applied from the start; the unit fallback contributes exp2(0 - m).
 * It is also the definition the HIP path uses for the rows it classifies as dense
 * (orc_dense_row below). */
static void direct_forward_row(const float* sq, const float* sk, const float* v,
                               const int32_t* q, const int32_t* k, const float* tab, int b,
                               int h, long N, int H, int R, int DV, float* out, float* lse2,
                               int32_t* lmax, int32_t* jarg, const int32_t* wlo) {
    /* lb[j+1] = L[i,j]; la[j] = L[i-1,j-1] */
    int32_t* la = (int32_t*)calloc((size_t)N + 1, sizeof(int32_t));
    int32_t* lb = (int32_t*)calloc((size_t)N + 1, sizeof(int32_t));
    float* acc = (float*)malloc(sizeof(float) * (size_t)DV);
    for (long i = 0; i < N; ++i) {
        long row = ((long)b * N + i) * H + h;
        float* o = out + row * DV;
        const int reset = wlo && wlo[i] == i;
        float m = 0.0f;
        int32_t best = 0, bj = -1;
        for (long j = 0; j <= i; ++j) {
            if (q[i] != k[j]) { lb[j + 1] = 0; continue; }
            int32_t L = reset ? 1 : la[j] + 1;
            lb[j + 1] = L;
            if (L >= best) { best = L; bj = (int32_t)j; }
            if (tab[L] > m) m = tab[L];
        }
        float den = orc_exp2f(-m);
        for (int d = 0; d < DV; ++d) acc[d] = 0.0f;
        const float* sqi = sq + row * R;
        for (long j = 0; j <= i; ++j) {
            int32_t L = lb[j + 1];
            if (!L) continue;
            float p = orc_exp2f(tab[L] - m);
            den = den + p;
            long krow = ((long)b * N + j) * H + h;
            const float* skj = sk + krow * R;
            float s = 0.0f;
            for (int r = 0; r < R; ++r) s = fmaf(sqi[r], skj[r], s);
            float ps = p * s;
            const float* vj = v + krow * DV;
            for (int d = 0; d < DV; ++d) acc[d] = fmaf(ps, vj[d], acc[d]);
        }
        for (int d = 0; d < DV; ++d) o[d] = acc[d] / den;
        lse2[i] = m + orc_log2f(den);
        if (lmax) lmax[i] = best;
        if (jarg) jarg[i] = bj;
        int32_t* t = la; la = lb; lb = t;
    }
    free(la);
    free(lb);
    free(acc);
}

static void zero_forward_row(int b, int h, long N, int H, int DV, float* out, float* lse2,
                             int32_t* lmax, int32_t* jarg) {
    for (long i = 0; i < N; ++i) {
        long row = ((long)b * N + i) * H + h;
        for (int d = 0; d < DV; ++d) out[row * DV + d] = 0.0f;
        lse2[i] = 0.0f;
        if (lmax) lmax[i] = 0;
        if (jarg) jarg[i] = -1;
    }
}

void orc_forward_direct(const float* sq, const float* sk, const float* v, const int32_t* iq,
                 const int32_t* ik, const uint8_t* hard, const float* lut, long lut_stride,
                 int B, long N, int H, int R, int DV, float* out, float* lse2, int32_t* lmax,
                 int32_t* jarg, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int bh = 0; bh < B * H; ++bh) {
        int b = bh / H, h = bh % H;
        long so = (long)bh * N;
        if (!hard[bh]) {
            zero_forward_row(b, h, N, H, DV, out, lse2 + so, lmax ? lmax + so : NULL,
                             jarg ? jarg + so : NULL);
            continue;
        }
        direct_forward_row(sq, sk, v, iq + so, ik + so, lut + (long)h * lut_stride, b, h, N, H,
                           R, DV, out, lse2 + so, lmax ? lmax + so : NULL,
                           jarg ? jarg + so : NULL, NULL);
    }
}

/* ---------------- direct backward ----------------
 * Row-major traversal (i ascending, j ascending) gives every per-key accumulator its
 * ascending-i order and every per-row accumulator its ascending-j order:
 *   p = exp2(LUT[L]-lse2_i); s = sq_i.sk_j; e = dO_i.v_j (fma chains)
 *   ps=p*s; pe=p*e; pse=ps*e; g = G[L]-G[i+1]
 *   dsq_i += pe*sk_j; dsk_j += pe*sq_i; dv_j += ps*dO_i
 *   u += pse; vv = fma(p,g,vv); w = fma(pse,g,w); z += p
 *   rowtau_i = (w - u*((vv - f c)/(z+f)))/(z+f),  f = exp2(-lse2_i), c = G[i+1]
 * dtau_h = sum over (b,i) of rowtau in the fixed blocked order of orc_tau_reduce.
 * The per-row outputs (dsq, dsk, dv of row (b,h), rowtau) must be zero on entry. */
static void direct_backward_row(const float* sq, const float* sk, const float* v,
                                const float* dout, const int32_t* q, const int32_t* k,
                                const float* tab, const float* gt, const float* l2v, int b,
                                int h, long N, int H, int R, int DV, float* dsq, float* dsk,
                                float* dv, float* rowtau) {
    int32_t* la = (int32_t*)calloc((size_t)N + 1, sizeof(int32_t));
    int32_t* lb = (int32_t*)calloc((size_t)N + 1, sizeof(int32_t));
    float* dq = (float*)malloc(sizeof(float) * (size_t)R);
    for (long i = 0; i < N; ++i) {
        long row = ((long)b * N + i) * H + h;
        const float* sqi = sq + row * R;
        const float* doi = dout + row * DV;
        float l2 = l2v[i];
        float c = gt[i + 1];
        float u = 0.0f, vv = 0.0f, w = 0.0f, z = 0.0f;
        for (int r = 0; r < R; ++r) dq[r] = 0.0f;
        for (long j = 0; j <= i; ++j) {
            if (q[i] != k[j]) { lb[j + 1] = 0; continue; }
            int32_t L = la[j] + 1;
            lb[j + 1] = L;
            float p = orc_exp2f(tab[L] - l2);
            long krow = ((long)b * N + j) * H + h;
            const float* skj = sk + krow * R;
            const float* vj = v + krow * DV;
            float s = 0.0f;
            for (int r = 0; r < R; ++r) s = fmaf(sqi[r], skj[r], s);
            float e = 0.0f;
            for (int d = 0; d < DV; ++d) e = fmaf(doi[d], vj[d], e);
            float ps = p * s, pe = p * e, pse = ps * e;
            float g = gt[L] - c;
            for (int r = 0; r < R; ++r) dq[r] = fmaf(pe, skj[r], dq[r]);
            float* dkj = dsk + krow * R;
            for (int r = 0; r < R; ++r) dkj[r] = fmaf(pe, sqi[r], dkj[r]);
            float* dvj = dv + krow * DV;
            for (int d = 0; d < DV; ++d) dvj[d] = fmaf(ps, doi[d], dvj[d]);
            u = u + pse;
            vv = fmaf(p, g, vv);
            w = fmaf(pse, g, w);
            z = z + p;
        }
        for (int r = 0; r < R; ++r) dsq[row * R + r] = dq[r];
        float f = orc_exp2f(-l2);
        float mass = z + f;
        float mean = fmaf(-f, c, vv) / mass;
        rowtau[i] = fmaf(-u, mean, w) / mass;
        int32_t* t = la; la = lb; lb = t;
    }
    free(la);
    free(lb);
    free(dq);
}

static void zero_backward_row(int b, int h, long N, int H, int R, int DV, float* dsq,
                              float* dsk, float* dv, float* rowtau) {
    for (long x = 0; x < N; ++x) {
        long row = ((long)b * N + x) * H + h;
        for (int r = 0; r < R; ++r) { dsq[row * R + r] = 0.0f; dsk[row * R + r] = 0.0f; }
        for (int d = 0; d < DV; ++d) dv[row * DV + d] = 0.0f;
        rowtau[x] = 0.0f;
    }
}

void orc_backward_direct(const float* sq, const float* sk, const float* v, const float* dout,
                  const int32_t* iq, const int32_t* ik, const uint8_t* hard, const float* lut,
                  const float* dlut, long lut_stride, const float* lse2in, int B, long N, int H,
                  int R, int DV, float* dsq, float* dsk, float* dv, float* rowtau, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int bh = 0; bh < B * H; ++bh) {
        int b = bh / H, h = bh % H;
        long so = (long)bh * N;
        zero_backward_row(b, h, N, H, R, DV, dsq, dsk, dv, rowtau + so);
        if (!hard[bh]) continue;
        direct_backward_row(sq, sk, v, dout, iq + so, ik + so, lut + (long)h * lut_stride,
                            dlut + (long)h * lut_stride, lse2in + so, b, h, N, H, R, DV, dsq,
                            dsk, dv, rowtau + so);
    }
}

/* ---------------- dense-row classification ----------------
 * The HIP path computes a hard row with the direct definition above ("dense" row) when its
 * labels collide often:
 *   M = sum over 4096 label buckets of (#queries in the bucket) * (#keys in the bucket),
 *   bucket(label) = ((uint32)label * 0x9E3779B1) >> 20 (the top 12 bits of a multiplicative
 *   hash), dense iff 64 * M > N^2 and N <= DENSE_MAX_N (its match-length boundaries are
 *   16-bit).
 * M is at least the exact collision count W = sum over labels of #queries * #keys (equal
 * labels share a bucket) and exceeds it only by bucket sharing (~N^2/4096 for many distinct
 * labels).  Dense rows have Theta(N^2) valid pairs; the decomposed definition's label scans
 * and bigram walks would be serial in the largest label group, or cubic in N, there.  Random
 * 256-symbol labels give M ~ N^2 / 256.  Soft rows are never dense. */
#define DENSE_MAX_N 65536L
#define DENSE_BUCKETS 4096

static inline uint32_t label_bucket(int32_t label) {
    return ((uint32_t)label * 0x9E3779B1u) >> 20;
}

uint64_t orc_bucket_collisions(const int32_t* q, const int32_t* k, long N) {
    uint64_t cq[DENSE_BUCKETS], ck[DENSE_BUCKETS];
    memset(cq, 0, sizeof(cq));
    memset(ck, 0, sizeof(ck));
    for (long x = 0; x < N; ++x) {
        cq[label_bucket(q[x])]++;
        ck[label_bucket(k[x])]++;
    }
    uint64_t m = 0;
    for (int b = 0; b < DENSE_BUCKETS; ++b) m += cq[b] * ck[b];
    return m;
}

int orc_dense_row(const int32_t* q, const int32_t* k, long N, int hard) {
    if (!hard || N > DENSE_MAX_N) return 0;
    return orc_bucket_collisions(q, k, N) * 64u > (uint64_t)N * (uint64_t)N;
}

void orc_dense_rows(const int32_t* iq, const int32_t* ik, const uint8_t* hard, int BH, long N,
                    uint8_t* dense) {
    for (int bh = 0; bh < BH; ++bh)
        dense[bh] = (uint8_t)orc_dense_row(iq + (long)bh * N, ik + (long)bh * N, N, hard[bh]);
}

/* ---------------- level rows ----------------
 * A dense row whose labels are all below 256, with N <= LEVEL_MAX_N, R * DV <= LEVEL_RDV, no
 * query resets, and whose longest match is at most LEVEL_MAX (with at most LEVEL_BUDGET * N
 * kept entries over all levels, below) is a "level row".  Its sums are taken per match
 * length instead of per pair.
 *
 * Level l groups the 2N entries e = 2p + s (s = 0 key, 1 query at position p, p >= l - 1) by
 * their l-gram (label[p - l + 1], ..., label[p]); a valid pair (j <= i) has L >= l exactly
 * when key j and query i share a level-l group.  The level-l list is the level-(l-1) kept
 * list without its entries at p = l - 2, stably sorted by label[p - l + 1] (level 1: all
 * entries in e order, sorted by label): inside a group the entries stay in e order (a key
 * before the query of its position).  A group is kept when one of its queries has a key
 * before it; the others cannot hold a valid pair at this or any deeper level.  The levels
 * stop at the first level with no kept group.
 *
 * Per query i and level l <= Lq (Lq = the longest match of i, lmax): n_l = keys before it in
 * its group (the valid keys with L >= l); y_l = sq_i . M_l with M_l = sum over those keys
 * of sk_j (x) v_j.  With p_l = exp2(LUT[l] - m), p_0 = 0, c_l = p_l - p_{l-1}:
 *   sum over valid j of p(L_ij) x_j = sum over l of c_l * (sum over keys with L >= l of x_j).
 * m = max(0, LUT[l] over the lengths l present, n_l > n_{l+1}), as the direct definition's.
 *
 * M_l comes from segments of LEVEL_SEG consecutive list entries: a query's M starts from the
 * prefix P_s of its segment (when its group began in an earlier segment, else from zero) and
 * runs an fma chain over the keys of its group before it in the segment.  T_s (the chain over
 * the keys of a segment's last group piece when that group continues into the next segment)
 * and P_{s+1} = P_s + T_s (P_{s+1} = T_s when the group began inside segment s) give the
 * prefixes.  The backward's key side runs the mirror image over queries in descending order
 * (U_s over the first piece, Q_{s-1} = Q_s + U_s).
 *
 * fp32 sequences (the HIP kernels of dism_levels.hip compute exactly these):
 *   forward, query i: m as above; den = exp2(-m); for l = 1..Lq: den = fma(c_l, n_l, den);
 *     acc[d] = fma(c_l, y_l[d], acc[d]) (acc from +0); y_l[d] = chain_r fma(sq[r], M[r][d]);
 *     out = acc / den, lse2 = m + log2(den); jarg = the last key of i's level-Lq group before it.
 *   backward, query i (p_l from l2 = lse2_i, cc = G[i + 1], F_l = p_l * (G[l] - cc), F_0 = 0,
 *     dF_l = F_l - F_{l-1}): z_l[r] = lane tree of dO[d] * M[r][d] (level_tree),
 *     w_l = chain_r fma(sq[r], z_l[r]); dq[r] = fma(c_l, z_l[r], dq[r]); u = fma(c_l, w_l, u);
 *     vv = fma(dF_l, n_l, vv); ww = fma(dF_l, w_l, ww); z = fma(c_l, n_l, z); then rowtau
 *     as the direct definition's.
 *   backward, key j, levels l = 1..(its kept levels): K[d][r] = fma(a_i[r], dO_i[d], K) over
 *     the queries after it in its group piece, descending, from Q_s or zero, a_i[r] =
 *     c_l(i) * sq_i[r]; dv_l[d] = chain_r fma(sk[r], K[d][r]); dk_l[r] = level_tree of
 *     v[d] * K[d][r]; dv = dv_1 + dv_2 + ..., dk likewise (left to right). */
static float dot_chain(const float* a, const float* b, int n);

#define LEVEL_MAX_N 4096L
#define LEVEL_MAX 32
#define LEVEL_BUDGET 16L
#define LEVEL_SEG 32L
#define LEVEL_RDV 512
#define LEVEL_START 0x40000000

typedef struct {
    int nlev;
    long off[LEVEL_MAX + 2];  /* level l (1-based) entries at [off[l-1], off[l]) */
    int32_t* ent;             /* e | LEVEL_START at a group's first entry */
} Levels;

/* 1 (and L filled; free L->ent) when the labels make a level row; the caller checks N, R*DV
 * and the absence of resets */
static int levels_build(const int32_t* q, const int32_t* k, long N, Levels* L) {
    L->ent = NULL;
    L->nlev = 0;
    if (N < 1 || N > LEVEL_MAX_N) return 0;
    for (long x = 0; x < N; ++x)
        if ((uint32_t)q[x] >= 256u || (uint32_t)k[x] >= 256u) return 0;
    const long M2 = 2 * N, cap = LEVEL_BUDGET * N;
    int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* cg = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* in = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* ig = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* id = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* se = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* sg = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* sd = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    L->ent = (int32_t*)malloc(sizeof(int32_t) * (size_t)cap);
    long m = M2, total = 0;
    int ok = 0;
    for (long e = 0; e < M2; ++e) { cur[e] = (int32_t)e; cg[e] = 0; }
    L->off[0] = 0;
    for (int l = 1; l <= LEVEL_MAX + 1; ++l) {
        long mi = 0;
        for (long t = 0; t < m; ++t) {
            const int32_t e = cur[t] & ~LEVEL_START;
            const long p = e >> 1;
            if (p < l - 1) continue;
            in[mi] = e;
            ig[mi] = cg[t];
            id[mi] = ((e & 1) ? q : k)[p - l + 1];
            ++mi;
        }
        long cnt[257];
        memset(cnt, 0, sizeof(cnt));
        for (long t = 0; t < mi; ++t) cnt[id[t] + 1]++;
        for (int d = 0; d < 256; ++d) cnt[d + 1] += cnt[d];
        for (long t = 0; t < mi; ++t) {
            const long dst = cnt[id[t]]++;
            se[dst] = in[t];
            sg[dst] = ig[t];
            sd[dst] = id[t];
        }
        long om = 0;
        for (long t = 0; t < mi;) {
            long te = t + 1;
            while (te < mi && sd[te] == sd[t] && sg[te] == sg[t]) ++te;
            int nk = 0, keep = 0;
            for (long x = t; x < te; ++x) {
                if (!(se[x] & 1)) ++nk;
                else if (nk > 0) keep = 1;
            }
            if (keep) {
                if (l <= LEVEL_MAX && total + om + (te - t) <= cap)
                    for (long x = t; x < te; ++x) {
                        L->ent[total + om + (x - t)] = se[x] | (x == t ? LEVEL_START : 0);
                        cg[om + (x - t)] = (int32_t)om;  /* next level's group id */
                    }
                om += te - t;
            }
            t = te;
        }
        if (om == 0) { L->nlev = l - 1; ok = 1; break; }
        if (l == LEVEL_MAX + 1 || total + om > cap) break;
        for (long x = 0; x < om; ++x) cur[x] = L->ent[total + x];
        m = om;
        total += om;
        L->off[l] = total;
    }
    free(cur); free(cg); free(in); free(ig); free(id); free(se); free(sg); free(sd);
    if (!ok) { free(L->ent); L->ent = NULL; }
    return ok;
}

/* the row's level count (>= 1), or 0 when it is not a level row (dense or not) */
int orc_level_row(const int32_t* q, const int32_t* k, long N, int R, int DV) {
    if ((long)R * DV > LEVEL_RDV) return 0;
    if (!orc_dense_row(q, k, N, 1)) return 0;
    Levels L;
    if (!levels_build(q, k, N, &L)) return 0;
    free(L.ent);
    return L.nlev;
}

/* ---------------- prefix rows ----------------
 * A hard row is a prefix row when it is dense (orc_dense_row), has no query resets, and
 * every label has one predecessor label: for all positions p, p' >= 1 on either side whose
 * labels are equal, the labels at p - 1 and p' - 1 (on the same sides) are equal too
 * (all-identical labels, a period of distinct labels; checked per label bucket,
 * prefix_labels).  Then a valid pair (i, j <= i,
 * iq[i] == ik[j]) with j >= 1 has iq[i-1] == ik[j-1], and by induction on j its match
 * reaches the key's row start: L_ij = j + 1.  The weight exp2(LUT[j+1] - m) of a pair is
 * then a function of the key, and a query's sum over its valid keys is a prefix sum over
 * its label group -- with a running maximum, because LUT[j+1] grows with j past the fp32
 * range of exp2 on long rows.
 *
 * The list is the combined label order: the 2N entries e = 2p + s (s = 0 key, 1 query at
 * position p) sorted by (label, p, s), so a label group is a run of entries and a query's
 * valid keys are the keys before it in its run.  Segments of PREFIX_SEG entries.  With
 * l_t = LUT[p_t + 1] for a key entry t:
 *
 * forward, per segment s:  over the keys t of its last piece (the entries of the group of
 *   its last entry that lie in s), ascending: M_s = max l_t; w = exp2(l_t - M_s);
 *   T_s[r][d] = fma(w * sk_t[r], v_t[d], T_s[r][d]); S_s = S_s + w; K_s = p of the last key.
 * prefix chain, s ascending, state (mu = 0, P = 0, PS = 0, lk = -1):  Pre_s = state; when
 *   the last piece's group starts in s (at or after its first entry) the state restarts;
 *   when the piece has keys: mu' = max(mu, M_s), g = exp2(mu - mu'), h = exp2(M_s - mu'),
 *   P[e] = fma(h, T_s[e], P[e] * g), PS = fma(h, S_s, PS * g), mu = mu', lk = K_s.
 * query at entry x of segment s: it starts from Pre_s when its group began before s, else
 *   from the empty state; its own keys are those of its group in s before it.
 *   m = max(mu, l_t over its own keys); f = exp2(mu - m);
 *   y[d] = (chain_r fma(sq[r], P[r][d])) * f (0 from the empty state);
 *   den = fma(PS, f, exp2(-m)); own keys ascending: p = exp2(l_t - m); den = den + p;
 *   s = chain_r fma(sq[r], sk_t[r]); y[d] = fma(p * s, v_t[d], y[d]);
 *   out = y / den; lse2 = m + log2(den); jarg = its last valid key (own, else lk); lmax =
 *   jarg + 1 (0 with no key).
 *
 * backward, query side (l2 = lse2_i, c = G[i + 1], G the d ln W / d tau table): the same
 *   segments and chain carry also sums weighted by G - G0_s, centred on the G of the piece's
 *   last key (G grows like L, so uncentred sums would cancel): TB_s[r][d] =
 *   fma((w * (G_t - G0_s)) * sk_t[r], v_t[d], .), SG_s = fma(w, G_t - G0_s, .); the chain
 *   recentres its state first: PB[e] = fma(h, TB_s[e], fma(gam - G0_s, P[e], PB[e]) * g),
 *   PSG = fma(h, SG_s, fma(gam - G0_s, PS, PSG) * g), gam = G0_s.  kappa = exp2(mu - l2);
 *   zP[r] = lane_reduce(dO, P[r]), zB[r] = lane_reduce(dO, PB[r]) (0 from the empty state);
 *   dq[r] = zP[r] * kappa;  u0 = wave_tree(sq[r] * zP[r]) * kappa,
 *   W0 = wave_tree(sq[r] * zB[r]) * kappa (term r on lane r * 64/R);  z0 = PS * kappa;
 *   cg = c - gam; vv0 = fma(-cg, z0, PSG * kappa); w0 = fma(-cg, u0, W0).  Own keys, lane = entry slot in
 *   the segment: p = exp2(l_t - l2); s = chain_r(sq . sk_t); e = chain_d(dO . v_t);
 *   ps = p * s; pe = p * e; pse = ps * e; g = G_t - c;  u = u0 + wave_tree(pse),
 *   vv = vv0 + wave_tree(p * g), w = w0 + wave_tree(pse * g), z = z0 + wave_tree(p),
 *   dq[r] = dq[r] + lane_tree(pe * sk_t[r]);  rowtau as the direct definition's.
 * backward, key side, per segment s: over the queries of its first piece (the entries of the
 *   group of its first entry that lie in s), descending: lam_s = min l2_i;
 *   w = exp2(lam_s - l2_i); U_s[r][d] = fma(w * sq_i[r], dO_i[d], U_s[r][d]).
 *   suffix chain, s descending, state (none):  Suf_s = state; when the first piece's group
 *   ends in s the state restarts; when the piece has queries: the first sets (nu = lam_s,
 *   Q = U_s), later ones nu' = min(nu, lam_s), g = exp2(nu' - nu), h = exp2(nu' - lam_s),
 *   Q[e] = fma(h, U_s[e], Q[e] * g), nu = nu'.
 *   key at entry x of s: from Suf_s when its group continues past s: phi = exp2(l_j - nu),
 *   dv[d] = (chain_r fma(sk[r], Q[r][d])) * phi, dk[r] = lane_reduce(v, Q[r]) * phi (else
 *   0); own queries (its group's queries after it in s), lane = slot:
 *   p = exp2(l_j - l2_i); s, e, ps, pe as above; dk[r] = dk[r] + lane_tree(pe * sq_i[r]);
 *   ascending: dv[d] = fma(ps, dO_i[d], dv[d]).
 * wave_tree: xor butterfly t[l] = t[l] + t[l ^ o], o = 32, ..., 1, over 64 lanes (0 where no
 * term); lane_tree: lane_reduce's order over per-lane terms.
 * These are the sums of the reference's readout (dism_v3/include/forward/readout.cuh:16-61,
 * online maximum from 0 and unit fallback) and of its backward with the four-moment tau terms
 * (dism_v3/src/hard_backward.cu:26-154, 156-197), which the reference takes pair by pair
 * over every causal pair of these rows; only the association differs (pinned against
 * direct_forward_row / direct_backward_row and FP64 in tests/test_prefix_rows.py). */
#define PREFIX_SEG 64L

static float lane_reduce(const float* a, const float* b, int DV, int R);

/* 1 when every label bucket (label_bucket, the classification's hash) holds one label over
 * both sides and one predecessor label over the positions >= 1 of both sides -- every label
 * then has one predecessor label.  (A row whose distinct labels share a bucket is not taken,
 * whatever its predecessors: the HIP check keeps one slot per bucket.) */
static int prefix_labels(const int32_t* q, const int32_t* k, long N) {
    uint64_t* lab = (uint64_t*)calloc(4096, sizeof(uint64_t));
    uint64_t* pred = (uint64_t*)calloc(4096, sizeof(uint64_t));
    int ok = 1;
    for (long p = 0; p < N && ok; ++p)
        for (int side = 0; side < 2 && ok; ++side) {
            const int32_t* L = side ? k : q;
            const uint32_t b = label_bucket(L[p]);
            const uint64_t t = (1ull << 32) | (uint32_t)L[p];
            if (!lab[b]) lab[b] = t;
            else if (lab[b] != t) ok = 0;
            if (p >= 1 && ok) {
                const uint64_t u = (1ull << 32) | (uint32_t)L[p - 1];
                if (!pred[b]) pred[b] = u;
                else if (pred[b] != u) ok = 0;
            }
        }
    free(lab);
    free(pred);
    return ok;
}

int orc_prefix_row(const int32_t* q, const int32_t* k, long N) {
    return orc_dense_row(q, k, N, 1) && prefix_labels(q, k, N);
}

static int cmp_entry(const void* a, const void* b, void* ctx) {
    const int32_t* const* lab = (const int32_t* const*)ctx;
    const int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    const uint32_t lx = (uint32_t)lab[x & 1][x >> 1], ly = (uint32_t)lab[y & 1][y >> 1];
    if (lx != ly) return lx < ly ? -1 : 1;
    return x < y ? -1 : x > y;
}

/* the combined label order E[2N] and, per entry, its group's start gs and end ge */
static void prefix_list(const int32_t* q, const int32_t* k, long N, int32_t* E, int32_t* gs,
                        int32_t* ge) {
    const int32_t* lab[2] = {k, q};
    const long M2 = 2 * N;
    for (long e = 0; e < M2; ++e) E[e] = (int32_t)e;
    qsort_r(E, (size_t)M2, sizeof(int32_t), cmp_entry, (void*)lab);
    for (long x = 0; x < M2; ++x) {
        const int same = x > 0 && lab[E[x] & 1][E[x] >> 1] == lab[E[x - 1] & 1][E[x - 1] >> 1];
        gs[x] = same ? gs[x - 1] : (int32_t)x;
    }
    for (long x = M2 - 1; x >= 0; --x) {
        const int same = x + 1 < M2 &&
                         lab[E[x] & 1][E[x] >> 1] == lab[E[x + 1] & 1][E[x + 1] >> 1];
        ge[x] = same ? ge[x + 1] : (int32_t)(x + 1);
    }
}

/* xor-butterfly sum of 64 lane terms (lane 0's result; every lane's is the same) */
static float wave_tree(const float* t0) {
    float t[64], u[64];
    memcpy(t, t0, sizeof(t));
    for (int o = 32; o >= 1; o /= 2) {
        for (int l = 0; l < 64; ++l) u[l] = t[l] + t[l ^ o];
        memcpy(t, u, sizeof(t));
    }
    return t[0];
}

/* lane_reduce's order over 64 per-lane terms t[l] (read with stride st) */
static float lane_tree(const float* t0, long st, int R) {
    float t[64];
    const int G = 64 / R;
    for (int l = 0; l < 64; ++l) t[l] = t0[l * st];
    for (int m = 32; m >= G; m /= 2)
        for (int l = 0; l < m; ++l) t[l] = t[l] + t[l + m];
    for (int sz = 1; sz < G; sz *= 2)
        for (int g = 0; g < G; g += 2 * sz) t[g] = t[g] + t[g + sz];
    return t[0];
}

/* segment totals over each segment's last piece and the prefix chain, in place: on return
 * P[s] (and PB[s] when non-null), mu[s], PS[s], PSG[s], gam[s], lk[s] hold the state Pre_s */
static void prefix_chain(const int32_t* E, const int32_t* gs, long N, const float* tab,
                         const float* gt, const float* sk, const float* v, int b, int h,
                         int H, int R, int DV, float* P, float* PB, float* mu, float* PS,
                         float* PSG, float* gam, int32_t* lk) {
    const long M2 = 2 * N, nseg = (M2 + PREFIX_SEG - 1) / PREFIX_SEG, RD = (long)R * DV;
    float* T = (float*)malloc(sizeof(float) * (size_t)RD);
    float* TB = (float*)malloc(sizeof(float) * (size_t)RD);
    float* st = (float*)calloc((size_t)RD, sizeof(float));
    float* sb = (float*)calloc((size_t)RD, sizeof(float));
    float smu = 0.0f, sps = 0.0f, spsg = 0.0f, sgam = 0.0f;
    int32_t slk = -1;
    for (long s = 0; s < nseg; ++s) {
        const long x0 = s * PREFIX_SEG, end = x0 + PREFIX_SEG < M2 ? x0 + PREFIX_SEG : M2;
        const long lo = gs[end - 1] > x0 ? gs[end - 1] : x0;
        float M = 0.0f, S = 0.0f, SG = 0.0f;
        int has = 0;
        int32_t K = -1;
        for (long t = lo; t < end; ++t)
            if (!(E[t] & 1)) {
                const float l = tab[(E[t] >> 1) + 1];
                if (!has || l > M) M = l;
                has = 1;
            }
        for (long t = lo; t < end; ++t)
            if (!(E[t] & 1)) K = E[t] >> 1;
        const float G0 = PB && has ? gt[K + 1] : 0.0f;  /* the segment's centre */
        for (long e = 0; e < RD; ++e) { T[e] = 0.0f; TB[e] = 0.0f; }
        for (long t = lo; t < end; ++t) {
            if (E[t] & 1) continue;
            const long p = E[t] >> 1, row = ((long)b * N + p) * H + h;
            const float w = orc_exp2f(tab[p + 1] - M);
            const float dg = PB ? gt[p + 1] - G0 : 0.0f;
            const float wg = w * dg;
            for (int r = 0; r < R; ++r) {
                const float a = w * sk[row * R + r];
                for (int d = 0; d < DV; ++d)
                    T[(long)r * DV + d] = fmaf(a, v[row * DV + d], T[(long)r * DV + d]);
                if (PB) {
                    const float c = wg * sk[row * R + r];
                    for (int d = 0; d < DV; ++d)
                        TB[(long)r * DV + d] = fmaf(c, v[row * DV + d], TB[(long)r * DV + d]);
                }
            }
            S = S + w;
            if (PB) SG = fmaf(w, dg, SG);
        }
        /* Pre_s */
        memcpy(P + s * RD, st, sizeof(float) * (size_t)RD);
        if (PB) memcpy(PB + s * RD, sb, sizeof(float) * (size_t)RD);
        mu[s] = smu;
        PS[s] = sps;
        if (PSG) PSG[s] = spsg;
        if (gam) gam[s] = sgam;
        lk[s] = slk;
        if (gs[end - 1] >= x0) {
            smu = 0.0f; sps = 0.0f; spsg = 0.0f; sgam = 0.0f; slk = -1;
            for (long e = 0; e < RD; ++e) { st[e] = 0.0f; sb[e] = 0.0f; }
        }
        if (has) {
            const float m2 = M > smu ? M : smu;
            const float g = orc_exp2f(smu - m2), hh = orc_exp2f(M - m2);
            const float dG = sgam - G0;  /* recentre the state on this segment's centre */
            for (long e = 0; e < RD; ++e) {
                if (PB) sb[e] = fmaf(hh, TB[e], fmaf(dG, st[e], sb[e]) * g);
                st[e] = fmaf(hh, T[e], st[e] * g);
            }
            if (PB) spsg = fmaf(hh, SG, fmaf(dG, sps, spsg) * g);
            sps = fmaf(hh, S, sps * g);
            if (PB) sgam = G0;
            smu = m2;
            slk = K;
        }
    }
    free(T); free(TB); free(st); free(sb);
}

static void prefix_forward_row(const float* sq, const float* sk, const float* v,
                               const int32_t* q, const int32_t* k, const float* tab, int b,
                               int h, long N, int H, int R, int DV, float* out, float* lse2,
                               int32_t* lmax, int32_t* jarg) {
    const long M2 = 2 * N, nseg = (M2 + PREFIX_SEG - 1) / PREFIX_SEG, RD = (long)R * DV;
    int32_t* E = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* gs = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* ge = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    float* P = (float*)malloc(sizeof(float) * (size_t)(nseg * RD));
    float* mu = (float*)malloc(sizeof(float) * (size_t)nseg);
    float* PS = (float*)malloc(sizeof(float) * (size_t)nseg);
    int32_t* lk = (int32_t*)malloc(sizeof(int32_t) * (size_t)nseg);
    float* y = (float*)malloc(sizeof(float) * (size_t)DV);
    prefix_list(q, k, N, E, gs, ge);
    prefix_chain(E, gs, N, tab, NULL, sk, v, b, h, H, R, DV, P, NULL, mu, PS, NULL, NULL, lk);
    for (long x = 0; x < M2; ++x) {
        if (!(E[x] & 1)) continue;
        const long i = E[x] >> 1, s = x / PREFIX_SEG, x0 = s * PREFIX_SEG;
        const long row = ((long)b * N + i) * H + h;
        const int use = gs[x] < x0;
        const long lo = use ? x0 : gs[x];
        const float bmu = use ? mu[s] : 0.0f, bps = use ? PS[s] : 0.0f;
        int32_t jb = use ? lk[s] : -1;
        float m = bmu;
        for (long t = lo; t < x; ++t)
            if (!(E[t] & 1) && tab[(E[t] >> 1) + 1] > m) m = tab[(E[t] >> 1) + 1];
        const float f = orc_exp2f(bmu - m);
        const float* sqi = sq + row * R;
        for (int d = 0; d < DV; ++d) {
            float a = 0.0f;
            if (use)
                for (int r = 0; r < R; ++r) a = fmaf(sqi[r], P[s * RD + (long)r * DV + d], a);
            y[d] = a * f;
        }
        float den = fmaf(bps, f, orc_exp2f(-m));
        for (long t = lo; t < x; ++t) {
            if (E[t] & 1) continue;
            const long j = E[t] >> 1, krow = ((long)b * N + j) * H + h;
            const float p = orc_exp2f(tab[j + 1] - m);
            den = den + p;
            const float ps = p * dot_chain(sqi, sk + krow * R, R);
            for (int d = 0; d < DV; ++d) y[d] = fmaf(ps, v[krow * DV + d], y[d]);
            jb = (int32_t)j;
        }
        for (int d = 0; d < DV; ++d) out[row * DV + d] = y[d] / den;
        lse2[i] = m + orc_log2f(den);
        if (lmax) lmax[i] = jb >= 0 ? jb + 1 : 0;
        if (jarg) jarg[i] = jb;
    }
    free(E); free(gs); free(ge); free(P); free(mu); free(PS); free(lk); free(y);
}

static void prefix_backward_row(const float* sq, const float* sk, const float* v,
                                const float* dout, const int32_t* q, const int32_t* k,
                                const float* tab, const float* gt, const float* l2v, int b,
                                int h, long N, int H, int R, int DV, float* dsq, float* dsk,
                                float* dv, float* rowtau) {
    const long M2 = 2 * N, nseg = (M2 + PREFIX_SEG - 1) / PREFIX_SEG, RD = (long)R * DV;
    const int G = 64 / R;
    int32_t* E = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* gs = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    int32_t* ge = (int32_t*)malloc(sizeof(int32_t) * (size_t)M2);
    float* P = (float*)malloc(sizeof(float) * (size_t)(nseg * RD));
    float* PB = (float*)malloc(sizeof(float) * (size_t)(nseg * RD));
    float* Q = (float*)malloc(sizeof(float) * (size_t)(nseg * RD));
    float* mu = (float*)malloc(sizeof(float) * (size_t)nseg);
    float* PS = (float*)malloc(sizeof(float) * (size_t)nseg);
    float* PSG = (float*)malloc(sizeof(float) * (size_t)nseg);
    float* gam = (float*)malloc(sizeof(float) * (size_t)nseg);
    float* nu = (float*)malloc(sizeof(float) * (size_t)nseg);
    uint8_t* qh = (uint8_t*)malloc((size_t)nseg);
    int32_t* lk = (int32_t*)malloc(sizeof(int32_t) * (size_t)nseg);
    float* U = (float*)malloc(sizeof(float) * (size_t)RD);
    float* st = (float*)calloc((size_t)RD, sizeof(float));
    float* X = (float*)malloc(sizeof(float) * (size_t)(64 * R));
    float *zP = (float*)malloc(sizeof(float) * (size_t)R), *zB = (float*)malloc(sizeof(float) * (size_t)R);
    float* col = (float*)malloc(sizeof(float) * (size_t)DV);
    prefix_list(q, k, N, E, gs, ge);
    prefix_chain(E, gs, N, tab, gt, sk, v, b, h, H, R, DV, P, PB, mu, PS, PSG, gam, lk);
    /* ---- query side */
    for (long x = 0; x < M2; ++x) {
        if (!(E[x] & 1)) continue;
        const long i = E[x] >> 1, s = x / PREFIX_SEG, x0 = s * PREFIX_SEG;
        const long row = ((long)b * N + i) * H + h;
        const float* sqi = sq + row * R;
        const float* doi = dout + row * DV;
        const float l2 = l2v[i], c = gt[i + 1];
        const int use = gs[x] < x0;
        const long lo = use ? x0 : gs[x];
        const float kap = orc_exp2f((use ? mu[s] : 0.0f) - l2);
        float t1[64], t2[64];
        for (int r = 0; r < R; ++r) {
            if (use) {
                for (int d = 0; d < DV; ++d) col[d] = P[s * RD + (long)r * DV + d];
                zP[r] = lane_reduce(doi, col, DV, R);
                for (int d = 0; d < DV; ++d) col[d] = PB[s * RD + (long)r * DV + d];
                zB[r] = lane_reduce(doi, col, DV, R);
            } else {
                zP[r] = 0.0f;
                zB[r] = 0.0f;
            }
        }
        for (int l = 0; l < 64; ++l) { t1[l] = 0.0f; t2[l] = 0.0f; }
        for (int r = 0; r < R; ++r) { t1[r * G] = sqi[r] * zP[r]; t2[r * G] = sqi[r] * zB[r]; }
        const float u0 = wave_tree(t1) * kap, W0 = wave_tree(t2) * kap;
        const float z0 = (use ? PS[s] : 0.0f) * kap, zg0 = (use ? PSG[s] : 0.0f) * kap;
        const float cg = c - (use ? gam[s] : 0.0f);
        const float vv0 = fmaf(-cg, z0, zg0), w0 = fmaf(-cg, u0, W0);
        float A[64], Bt[64], C[64], D[64];
        for (int l = 0; l < 64; ++l) {
            A[l] = 0.0f; Bt[l] = 0.0f; C[l] = 0.0f; D[l] = 0.0f;
            for (int r = 0; r < R; ++r) X[l * R + r] = 0.0f;
            const long t = x0 + l;
            if (t < lo || t >= x || (E[t] & 1)) continue;
            const long j = E[t] >> 1, krow = ((long)b * N + j) * H + h;
            const float p = orc_exp2f(tab[j + 1] - l2);
            const float sv = dot_chain(sqi, sk + krow * R, R);
            const float ev = dot_chain(doi, v + krow * DV, DV);
            const float ps = p * sv, pe = p * ev, pse = ps * ev, g = gt[j + 1] - c;
            A[l] = pse; Bt[l] = p * g; C[l] = pse * g; D[l] = p;
            for (int r = 0; r < R; ++r) X[l * R + r] = pe * sk[krow * R + r];
        }
        const float u = u0 + wave_tree(A), vv = vv0 + wave_tree(Bt);
        const float w = w0 + wave_tree(C), z = z0 + wave_tree(D);
        for (int r = 0; r < R; ++r) dsq[row * R + r] = zP[r] * kap + lane_tree(X + r, R, R);
        const float f = orc_exp2f(-l2), mass = z + f;
        const float mean = fmaf(-f, c, vv) / mass;
        rowtau[i] = fmaf(-u, mean, w) / mass;
    }
    /* ---- key side: suffix chain over each segment's first piece */
    {
        int has = 0;
        float snu = 0.0f;
        for (long s = nseg - 1; s >= 0; --s) {
            const long x0 = s * PREFIX_SEG, end = x0 + PREFIX_SEG < M2 ? x0 + PREFIX_SEG : M2;
            const long hi = ge[x0] < end ? ge[x0] : end;
            float lam = 0.0f;
            int hu = 0;
            for (long t = x0; t < hi; ++t)
                if (E[t] & 1) {
                    const float l2 = l2v[E[t] >> 1];
                    if (!hu || l2 < lam) lam = l2;
                    hu = 1;
                }
            for (long e = 0; e < RD; ++e) U[e] = 0.0f;
            for (long t = hi - 1; t >= x0; --t) {
                if (!(E[t] & 1)) continue;
                const long i = E[t] >> 1, row = ((long)b * N + i) * H + h;
                const float wq = orc_exp2f(lam - l2v[i]);
                for (int r = 0; r < R; ++r) {
                    const float a = wq * sq[row * R + r];
                    for (int d = 0; d < DV; ++d)
                        U[(long)r * DV + d] = fmaf(a, dout[row * DV + d], U[(long)r * DV + d]);
                }
            }
            memcpy(Q + s * RD, st, sizeof(float) * (size_t)RD);
            nu[s] = snu;
            qh[s] = (uint8_t)has;
            if (ge[x0] <= end) {
                has = 0;
                snu = 0.0f;
                for (long e = 0; e < RD; ++e) st[e] = 0.0f;
            }
            if (hu) {
                if (!has) {
                    snu = lam;
                    memcpy(st, U, sizeof(float) * (size_t)RD);
                    has = 1;
                } else {
                    const float n2 = lam < snu ? lam : snu;
                    const float g = orc_exp2f(n2 - snu), hh = orc_exp2f(n2 - lam);
                    for (long e = 0; e < RD; ++e) st[e] = fmaf(hh, U[e], st[e] * g);
                    snu = n2;
                }
            }
        }
    }
    for (long x = 0; x < M2; ++x) {
        if (E[x] & 1) continue;
        const long j = E[x] >> 1, s = x / PREFIX_SEG, x0 = s * PREFIX_SEG;
        const long end = x0 + PREFIX_SEG < M2 ? x0 + PREFIX_SEG : M2;
        const long krow = ((long)b * N + j) * H + h;
        const float* skj = sk + krow * R;
        const float* vj = v + krow * DV;
        const float lj = tab[j + 1];
        const int use = ge[x] > end && qh[s];
        const long hi = ge[x] < end ? ge[x] : end;
        float* dkj = dsk + krow * R;
        float* dvj = dv + krow * DV;
        const float phi = use ? orc_exp2f(lj - nu[s]) : 0.0f;
        for (int d = 0; d < DV; ++d) {
            float a = 0.0f;
            if (use)
                for (int r = 0; r < R; ++r) a = fmaf(skj[r], Q[s * RD + (long)r * DV + d], a);
            dvj[d] = use ? a * phi : 0.0f;
        }
        for (int r = 0; r < R; ++r) {
            if (use) {
                for (int d = 0; d < DV; ++d) col[d] = Q[s * RD + (long)r * DV + d];
                dkj[r] = lane_reduce(vj, col, DV, R) * phi;
            } else {
                dkj[r] = 0.0f;
            }
        }
        for (int l = 0; l < 64; ++l) {
            for (int r = 0; r < R; ++r) X[l * R + r] = 0.0f;
            const long t = x0 + l;
            if (t <= x || t >= hi || !(E[t] & 1)) continue;
            const long i = E[t] >> 1, row = ((long)b * N + i) * H + h;
            const float p = orc_exp2f(lj - l2v[i]);
            const float ev = dot_chain(dout + row * DV, vj, DV);
            const float pe = p * ev;
            for (int r = 0; r < R; ++r) X[l * R + r] = pe * sq[row * R + r];
        }
        for (int r = 0; r < R; ++r) dkj[r] = dkj[r] + lane_tree(X + r, R, R);
        for (long t = x + 1; t < hi; ++t) {
            if (!(E[t] & 1)) continue;
            const long i = E[t] >> 1, row = ((long)b * N + i) * H + h;
            const float p = orc_exp2f(lj - l2v[i]);
            const float ps = p * dot_chain(sq + row * R, skj, R);
            for (int d = 0; d < DV; ++d) dvj[d] = fmaf(ps, dout[row * DV + d], dvj[d]);
        }
    }
    free(E); free(gs); free(ge); free(P); free(PB); free(Q); free(mu); free(PS); free(PSG); free(gam);
    free(nu); free(qh); free(lk); free(U); free(st); free(X); free(zP); free(zB); free(col);
}

/* row mode as the HIP path chooses it: 0 decomposed, 1 direct, 3 levels, 4 prefix */
static int row_mode(const int32_t* q, const int32_t* k, long N, int R, int DV, int resets) {
    if (!orc_dense_row(q, k, N, 1)) return 0;
    if (!resets && prefix_labels(q, k, N)) return 4;
    if (resets || (long)R * DV > LEVEL_RDV) return 1;
    Levels L;
    if (!levels_build(q, k, N, &L)) return 1;
    free(L.ent);
    return 3;
}

void orc_row_modes(const int32_t* iq, const int32_t* ik, int BH, long N, int R, int DV,
                   uint8_t* mode) {
    for (int bh = 0; bh < BH; ++bh)
        mode[bh] = (uint8_t)row_mode(iq + (long)bh * N, ik + (long)bh * N, N, R, DV, 0);
}

/* per (level, query or key position): index in the level list, -1 when not there; and
 * per query the key count before it in its group */
typedef struct {
    int32_t* idx;   /* [nlev][2N] by entry e */
    int32_t* nk;    /* [nlev][N] by query position */
    int32_t* lastk; /* [nlev][N] last key position before the query in its group, -1 */
} LevelMaps;

static void level_maps(const Levels* L, long N, LevelMaps* Mp) {
    const int nl = L->nlev;
    Mp->idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nl * 2 * N));
    Mp->nk = (int32_t*)calloc((size_t)(nl * N), sizeof(int32_t));
    Mp->lastk = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nl * N));
    for (long x = 0; x < nl * 2 * N; ++x) Mp->idx[x] = -1;
    for (long x = 0; x < nl * N; ++x) Mp->lastk[x] = -1;
    for (int l = 1; l <= nl; ++l) {
        const int32_t* E = L->ent + L->off[l - 1];
        const long m = L->off[l] - L->off[l - 1];
        int nk = 0, lk = -1;
        for (long t = 0; t < m; ++t) {
            if (E[t] & LEVEL_START) { nk = 0; lk = -1; }
            const int32_t e = E[t] & ~LEVEL_START;
            Mp->idx[(long)(l - 1) * 2 * N + e] = (int32_t)t;
            if (!(e & 1)) { ++nk; lk = e >> 1; }
            else {
                Mp->nk[(long)(l - 1) * N + (e >> 1)] = nk;
                Mp->lastk[(long)(l - 1) * N + (e >> 1)] = lk;
            }
        }
    }
}

static void level_maps_free(LevelMaps* Mp) { free(Mp->idx); free(Mp->nk); free(Mp->lastk); }

/* lane tree of per-lane terms: lane t (t < 64) holds a[t]*b[t] (t < DV), then
 * fma(a[t+64], b[t+64], .) (t + 64 < DV), else 0; t[l] = t[l] + t[l+m] for m = 32, ..., 1 */
static float level_tree(const float* a, long sa, const float* b, long sb, int DV) {
    float t[64];
    for (int l = 0; l < 64; ++l) {
        float x = l < DV ? a[l * sa] * b[l * sb] : 0.0f;
        if (l + 64 < DV) x = fmaf(a[(l + 64) * sa], b[(l + 64) * sb], x);
        t[l] = x;
    }
    for (int m = 32; m >= 1; m /= 2)
        for (int l = 0; l < m; ++l) t[l] = t[l] + t[l + m];
    return t[0];
}

/* forward prefixes of one level: P [nseg][R*DV], has [nseg] (1 when segment s's first
 * piece continues a group of an earlier segment) */
static void level_prefix(const Levels* L, int l, const float* sk, const float* v, int b, int h,
                         long N, int H, int R, int DV, float* P, uint8_t* has) {
    const int32_t* E = L->ent + L->off[l - 1];
    const long m = L->off[l] - L->off[l - 1], nseg = (m + LEVEL_SEG - 1) / LEVEL_SEG;
    const long RD = (long)R * DV;
    float* T = (float*)malloc(sizeof(float) * (size_t)RD);
    for (long s = 0; s < nseg; ++s) has[s] = 0;
    for (long s = 0; s + 1 < nseg; ++s) {
        const long beg = s * LEVEL_SEG, end = beg + LEVEL_SEG;
        if (E[end] & LEVEL_START) continue;  /* no group crosses into s + 1 */
        long ls = beg;
        for (long x = beg; x < end; ++x)
            if (E[x] & LEVEL_START) ls = x;
        for (long e = 0; e < RD; ++e) T[e] = 0.0f;
        for (long x = ls; x < end; ++x) {
            const int32_t e = E[x] & ~LEVEL_START;
            if (e & 1) continue;
            const long krow = ((long)b * N + (e >> 1)) * H + h;
            for (int r = 0; r < R; ++r)
                for (int d = 0; d < DV; ++d)
                    T[r * DV + d] = fmaf(sk[krow * R + r], v[krow * DV + d], T[r * DV + d]);
        }
        /* segment s wholly inside the group (first piece continuing, no start): add */
        const int chain = has[s] && ls == beg && !(E[beg] & LEVEL_START);
        for (long e = 0; e < RD; ++e)
            P[(s + 1) * RD + e] = chain ? P[s * RD + e] + T[e] : T[e];
        has[s + 1] = 1;
    }
    free(T);
}

/* M of query entry x of level l (list E), from the segment prefix */
static void level_query_m(const int32_t* E, long x, const float* P, const uint8_t* has,
                          const float* sk, const float* v, int b, int h, long N, int H, int R,
                          int DV, float* M) {
    const long RD = (long)R * DV, s = x / LEVEL_SEG, beg = s * LEVEL_SEG;
    long ps = beg;
    int start = 0;
    for (long t = beg; t <= x; ++t)
        if (E[t] & LEVEL_START) { ps = t; start = 1; }
    for (long e = 0; e < RD; ++e) M[e] = (!start && has[s]) ? P[s * RD + e] : 0.0f;
    for (long t = ps; t < x; ++t) {
        const int32_t e = E[t] & ~LEVEL_START;
        if (e & 1) continue;
        const long krow = ((long)b * N + (e >> 1)) * H + h;
        for (int r = 0; r < R; ++r)
            for (int d = 0; d < DV; ++d)
                M[r * DV + d] = fmaf(sk[krow * R + r], v[krow * DV + d], M[r * DV + d]);
    }
}

static void level_forward_row(const float* sq, const float* sk, const float* v,
                              const float* tab, int b, int h, long N, int H, int R, int DV,
                              const Levels* L, float* out, float* lse2, int32_t* lmax,
                              int32_t* jarg) {
    const int nl = L->nlev;
    const long RD = (long)R * DV;
    LevelMaps Mp;
    level_maps(L, N, &Mp);
    float** P = (float**)malloc(sizeof(float*) * (size_t)nl);
    uint8_t** has = (uint8_t**)malloc(sizeof(uint8_t*) * (size_t)nl);
    for (int l = 1; l <= nl; ++l) {
        const long m = L->off[l] - L->off[l - 1], nseg = (m + LEVEL_SEG - 1) / LEVEL_SEG;
        P[l - 1] = (float*)malloc(sizeof(float) * (size_t)(nseg * RD));
        has[l - 1] = (uint8_t*)malloc((size_t)nseg);
        level_prefix(L, l, sk, v, b, h, N, H, R, DV, P[l - 1], has[l - 1]);
    }
    float* M = (float*)malloc(sizeof(float) * (size_t)RD);
    float* acc = (float*)malloc(sizeof(float) * (size_t)DV);
    for (long i = 0; i < N; ++i) {
        const long row = ((long)b * N + i) * H + h;
        int Lq = 0;
        for (int l = 1; l <= nl; ++l)
            if (Mp.idx[(long)(l - 1) * 2 * N + 2 * i + 1] >= 0 && Mp.nk[(long)(l - 1) * N + i] > 0)
                Lq = l;
        float m = 0.0f;
        for (int l = 1; l <= Lq; ++l) {
            const int n1 = Mp.nk[(long)(l - 1) * N + i];
            const int n2 = l < Lq ? Mp.nk[(long)l * N + i] : 0;
            if (n1 > n2 && tab[l] > m) m = tab[l];
        }
        float den = orc_exp2f(-m), pp = 0.0f;
        for (int d = 0; d < DV; ++d) acc[d] = 0.0f;
        const float* sqi = sq + row * R;
        for (int l = 1; l <= Lq; ++l) {
            const float p = orc_exp2f(tab[l] - m);
            const float c = p - pp;
            pp = p;
            den = fmaf(c, (float)Mp.nk[(long)(l - 1) * N + i], den);
            const long x = Mp.idx[(long)(l - 1) * 2 * N + 2 * i + 1];
            level_query_m(L->ent + L->off[l - 1], x, P[l - 1], has[l - 1], sk, v, b, h, N, H, R,
                          DV, M);
            for (int d = 0; d < DV; ++d) {
                float y = 0.0f;
                for (int r = 0; r < R; ++r) y = fmaf(sqi[r], M[r * DV + d], y);
                acc[d] = fmaf(c, y, acc[d]);
            }
        }
        for (int d = 0; d < DV; ++d) out[row * DV + d] = acc[d] / den;
        lse2[i] = m + orc_log2f(den);
        if (lmax) lmax[i] = Lq;
        if (jarg) jarg[i] = Lq ? Mp.lastk[(long)(Lq - 1) * N + i] : -1;
    }
    for (int l = 0; l < nl; ++l) { free(P[l]); free(has[l]); }
    free(P); free(has); free(M); free(acc);
    level_maps_free(&Mp);
}

/* c_l of query position i (l2 its lse2) */
static float level_c(const float* tab, int l, float l2) {
    const float p = orc_exp2f(tab[l] - l2);
    return l > 1 ? p - orc_exp2f(tab[l - 1] - l2) : p - 0.0f;
}

static void level_backward_row(const float* sq, const float* sk, const float* v,
                               const float* dout, const float* tab, const float* gt,
                               const float* l2v, int b, int h, long N, int H, int R, int DV,
                               const Levels* L, float* dsq, float* dsk, float* dv,
                               float* rowtau) {
    const int nl = L->nlev;
    const long RD = (long)R * DV;
    LevelMaps Mp;
    level_maps(L, N, &Mp);
    float** P = (float**)malloc(sizeof(float*) * (size_t)nl);
    uint8_t** has = (uint8_t**)malloc(sizeof(uint8_t*) * (size_t)nl);
    float** Q = (float**)malloc(sizeof(float*) * (size_t)nl);
    uint8_t** hq = (uint8_t**)malloc(sizeof(uint8_t*) * (size_t)nl);
    float* U = (float*)malloc(sizeof(float) * (size_t)RD);
    float* a = (float*)malloc(sizeof(float) * (size_t)R);
    for (int l = 1; l <= nl; ++l) {
        const int32_t* E = L->ent + L->off[l - 1];
        const long m = L->off[l] - L->off[l - 1], nseg = (m + LEVEL_SEG - 1) / LEVEL_SEG;
        P[l - 1] = (float*)malloc(sizeof(float) * (size_t)(nseg * RD));
        has[l - 1] = (uint8_t*)malloc((size_t)nseg);
        level_prefix(L, l, sk, v, b, h, N, H, R, DV, P[l - 1], has[l - 1]);
        /* key-side suffixes: K layout [d][r] */
        Q[l - 1] = (float*)malloc(sizeof(float) * (size_t)(nseg * RD));
        hq[l - 1] = (uint8_t*)calloc((size_t)nseg, 1);
        for (long s = nseg - 1; s >= 1; --s) {
            const long beg = s * LEVEL_SEG;
            const long end = beg + LEVEL_SEG < m ? beg + LEVEL_SEG : m;
            if (E[beg] & LEVEL_START) continue;  /* no group crosses from s - 1 */
            long fe = end;
            for (long x = end - 1; x > beg; --x)
                if (E[x] & LEVEL_START) fe = x;
            for (long e = 0; e < RD; ++e) U[e] = 0.0f;
            for (long x = fe - 1; x >= beg; --x) {
                const int32_t e = E[x] & ~LEVEL_START;
                if (!(e & 1)) continue;
                const long i = e >> 1;
                const long row = ((long)b * N + i) * H + h;
                const float c = level_c(tab, l, l2v[i]);
                for (int r = 0; r < R; ++r) a[r] = c * sq[row * R + r];
                for (int d = 0; d < DV; ++d)
                    for (int r = 0; r < R; ++r)
                        U[d * R + r] = fmaf(a[r], dout[row * DV + d], U[d * R + r]);
            }
            const int chain = hq[l - 1][s] && fe == end && end < m;
            for (long e = 0; e < RD; ++e)
                Q[l - 1][(s - 1) * RD + e] = chain ? Q[l - 1][s * RD + e] + U[e] : U[e];
            hq[l - 1][s - 1] = 1;
        }
    }
    float* M = (float*)malloc(sizeof(float) * (size_t)RD);
    float* zl = (float*)malloc(sizeof(float) * (size_t)R);
    float* dq = (float*)malloc(sizeof(float) * (size_t)R);
    /* ---- query rows */
    for (long i = 0; i < N; ++i) {
        const long row = ((long)b * N + i) * H + h;
        const float* sqi = sq + row * R;
        const float* doi = dout + row * DV;
        int Lq = 0;
        for (int l = 1; l <= nl; ++l)
            if (Mp.idx[(long)(l - 1) * 2 * N + 2 * i + 1] >= 0 && Mp.nk[(long)(l - 1) * N + i] > 0)
                Lq = l;
        const float l2 = l2v[i];
        const float cc = gt[i + 1];
        float u = 0.0f, vv = 0.0f, ww = 0.0f, z = 0.0f, pp = 0.0f, fp = 0.0f;
        for (int r = 0; r < R; ++r) dq[r] = 0.0f;
        for (int l = 1; l <= Lq; ++l) {
            const float p = orc_exp2f(tab[l] - l2);
            const float c = p - pp;
            const float F = p * (gt[l] - cc);
            const float dF = F - fp;
            pp = p;
            fp = F;
            const long x = Mp.idx[(long)(l - 1) * 2 * N + 2 * i + 1];
            level_query_m(L->ent + L->off[l - 1], x, P[l - 1], has[l - 1], sk, v, b, h, N, H, R,
                          DV, M);
            for (int r = 0; r < R; ++r) zl[r] = level_tree(doi, 1, M + (long)r * DV, 1, DV);
            const float w = dot_chain(sqi, zl, R);
            const float fn = (float)Mp.nk[(long)(l - 1) * N + i];
            for (int r = 0; r < R; ++r) dq[r] = fmaf(c, zl[r], dq[r]);
            u = fmaf(c, w, u);
            vv = fmaf(dF, fn, vv);
            ww = fmaf(dF, w, ww);
            z = fmaf(c, fn, z);
        }
        for (int r = 0; r < R; ++r) dsq[row * R + r] = dq[r];
        const float f = orc_exp2f(-l2);
        const float mass = z + f;
        const float mean = fmaf(-f, cc, vv) / mass;
        rowtau[i] = fmaf(-u, mean, ww) / mass;
    }
    /* ---- keys */
    float* K = M;  /* [d][r] */
    float* dkl = dq;
    for (long j = 0; j < N; ++j) {
        const long krow = ((long)b * N + j) * H + h;
        const float* skj = sk + krow * R;
        const float* vj = v + krow * DV;
        for (int l = 1; l <= nl; ++l) {
            const long x = Mp.idx[(long)(l - 1) * 2 * N + 2 * j];
            if (x < 0) break;
            const int32_t* E = L->ent + L->off[l - 1];
            const long m = L->off[l] - L->off[l - 1];
            const long s = x / LEVEL_SEG, beg = s * LEVEL_SEG;
            const long end = beg + LEVEL_SEG < m ? beg + LEVEL_SEG : m;
            long pe = end;
            for (long t = end - 1; t > x; --t)
                if (E[t] & LEVEL_START) pe = t;
            const int cont = pe == end && end < m && !(E[end] & LEVEL_START);
            for (long e = 0; e < RD; ++e) K[e] = cont ? Q[l - 1][s * RD + e] : 0.0f;
            for (long t = pe - 1; t > x; --t) {
                const int32_t e = E[t] & ~LEVEL_START;
                if (!(e & 1)) continue;
                const long i = e >> 1;
                const long row = ((long)b * N + i) * H + h;
                const float c = level_c(tab, l, l2v[i]);
                for (int r = 0; r < R; ++r) a[r] = c * sq[row * R + r];
                for (int d = 0; d < DV; ++d)
                    for (int r = 0; r < R; ++r)
                        K[d * R + r] = fmaf(a[r], dout[row * DV + d], K[d * R + r]);
            }
            for (int r = 0; r < R; ++r) dkl[r] = level_tree(vj, 1, K + r, R, DV);
            for (int d = 0; d < DV; ++d) {
                float y = 0.0f;
                for (int r = 0; r < R; ++r) y = fmaf(skj[r], K[d * R + r], y);
                dv[krow * DV + d] = l == 1 ? y : dv[krow * DV + d] + y;
            }
            for (int r = 0; r < R; ++r)
                dsk[krow * R + r] = l == 1 ? dkl[r] : dsk[krow * R + r] + dkl[r];
        }
    }
    for (int l = 0; l < nl; ++l) { free(P[l]); free(has[l]); free(Q[l]); free(hq[l]); }
    free(P); free(has); free(Q); free(hq); free(U); free(a); free(M); free(zl); free(dq);
    level_maps_free(&Mp);
}

/* dtau_h: for each head, the B*N row terms in (b, i) order are cut into blocks of `block`
 * rows; each block is summed sequentially in double; the block sums are cut into groups of
 * `group` consecutive blocks, each group summed sequentially in double; the group sums are
 * summed sequentially in double; the result is rounded to float. */
void orc_tau_reduce(const float* rowtau, int B, int H, long N, long block, long group,
                    float* dtau) {
    for (int h = 0; h < H; ++h) {
        long total = (long)B * N;
        double outer = 0.0, mid = 0.0;
        long t = 0;  /* block index */
        for (long s = 0; s < total; s += block, ++t) {
            double inner = 0.0;
            for (long x = s; x < s + block && x < total; ++x) {
                long b = x / N, i = x % N;
                inner += (double)rowtau[((long)b * H + h) * N + i];
            }
            mid += inner;
            if ((t + 1) % group == 0 || s + block >= total) {
                outer += mid;
                mid = 0.0;
            }
        }
        dtau[h] = (float)outer;
    }
}

/* ======================================================================================
 * Decomposed definition (the one the HIP kernels compute bit for bit).
 *
 * Split of the valid pairs of a row i (keys j <= i with iq[i] == ik[j]):
 *   - every valid pair is first counted as a length-1 pair with weight p1 = exp2(LUT[1]-m);
 *   - a "bigram" pair (i >= 1, j >= 1, iq[i-1] == ik[j-1]) is exactly a pair with L >= 2;
 *     it adds the correction (p - p1).
 * The length-1 part factorises through the per-label prefix matrix
 *   M_i[r][d] = sum over valid keys j of sk_j[r] * v_j[d]   (fma chain, ascending j)
 * and the key-side suffix matrix
 *   N_j[r][d] = sum over valid queries i of (p1_i * sq_i[r]) * dO_i[d]   (descending i).
 * Mathematically this equals the direct sums (orc_forward_direct / orc_backward_direct);
 * only the fp32 association differs.
 * ====================================================================================== */

static int cmp_lab_pos(const void* a, const void* b, void* ctx) {
    const int32_t* lab = (const int32_t*)ctx;
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    uint32_t lx = (uint32_t)lab[x], ly = (uint32_t)lab[y];
    if (lx != ly) return lx < ly ? -1 : 1;
    return x < y ? -1 : (x > y);
}

/* positions 0..N-1 ordered by (unsigned label, position) */
static void sort_by_label(const int32_t* lab, long N, int32_t* out) {
    for (long x = 0; x < N; ++x) out[x] = (int32_t)x;
    qsort_r(out, (size_t)N, sizeof(int32_t), cmp_lab_pos, (void*)lab);
}

/* Row-group reduction of sum_d a[d]*b[d] over DV columns for readout width R: the columns
 * are cut into G = 64/R consecutive groups of VPL = DV/G; each group is an fma chain in
 * ascending d, then the G partials are added as a pairwise tree ((t0 + t1) + (t2 + t3)) + ...
 * This is the order of the HIP row-group lane layout (lane = r*G + g) with in-row DPP adds. */
static float rg_reduce(const float* a, const float* b, int DV, int R) {
    float t[64];
    const int G = 64 / R, V = DV / G;
    for (int g = 0; g < G; ++g) {
        float s = 0.0f;
        for (int x = 0; x < V; ++x) s = fmaf(a[g * V + x], b[g * V + x], s);
        t[g] = s;
    }
    for (int sz = 1; sz < G; sz *= 2)
        for (int g = 0; g < G; g += 2 * sz) t[g] = t[g] + t[g + sz];
    return t[0];
}

/* Lane-tree reduction of sum_d a[d]*b[d] (DV <= 128) for readout width R, G = 64/R: lane l
 * holds the term fma(a[l+64], b[l+64], a[l]*b[l]) (DV = 128), a[l]*b[l] (l < DV) or 0; the
 * high lane bits are paired first, t[l] = t[l] + t[l+m] for m = 32, 16, ..., G, then the G
 * remaining partials form the pairwise tree ((t0 + t1) + (t2 + t3)) + ...  This is the order
 * of the HIP column-layout reduction (lane = d) with its transposing butterfly. */
static float lane_reduce(const float* a, const float* b, int DV, int R) {
    float t[64];
    const int G = 64 / R;
    for (int l = 0; l < 64; ++l) {
        float x = l < DV ? a[l] * b[l] : 0.0f;
        if (l + 64 < DV) x = fmaf(a[l + 64], b[l + 64], x);
        t[l] = x;
    }
    for (int m = 32; m >= G; m /= 2)
        for (int l = 0; l < m; ++l) t[l] = t[l] + t[l + m];
    for (int sz = 1; sz < G; sz *= 2)
        for (int g = 0; g < G; g += 2 * sz) t[g] = t[g] + t[g + sz];
    return t[0];
}

/* Pairwise tree ((t0 + t1) + (t2 + t3)) + ... over the products t[d] = a[d]*b[d], n a power
 * of two <= 128: the bigram-pair DV-dot of the HIP pair kernels (lanes hold contiguous
 * column groups, reduced in-lane and then across lanes by the same adjacent pairing). */
static float tree_dot(const float* a, const float* b, int n) {
    float t[128];
    for (int d = 0; d < n; ++d) t[d] = a[d] * b[d];
    for (int sz = 1; sz < n; sz *= 2)
        for (int g = 0; g < n; g += 2 * sz) t[g] = t[g] + t[g + sz];
    return t[0];
}

static float dot_chain(const float* a, const float* b, int n) {
    float s = 0.0f;
    for (int r = 0; r < n; ++r) s = fmaf(a[r], b[r], s);
    return s;
}

/* lower bound of label value x in positions `ord` sorted by label */
static long label_lb(const int32_t* lab, const int32_t* ord, long N, uint32_t x) {
    long lo = 0, hi = N;
    while (lo < hi) {
        long mid = (lo + hi) / 2;
        if ((uint32_t)lab[ord[mid]] < x) lo = mid + 1; else hi = mid;
    }
    return lo;
}

/* Forward, per row i of a hard (b,h):
 *   cnt = #valid keys, last = largest valid key; pairs P = bigram pairs, ascending j, with
 *   L = suffix walk (>= 2);
 *   m = 0; if cnt>0 && LUT[1] > m: m = LUT[1]; for j in P: if LUT[L] > m: m = LUT[L]
 *   Lmax/jarg: P nonempty -> max L, ties to the largest j; else cnt>0 -> (1, last); else (0,-1)
 *   p1 = exp2(LUT[1]-m)
 *   for j in P: p = exp2(LUT[L]-m); dp = dp + p; s = chain(sq_i.sk_j); c = (p-p1)*s;
 *               corr[d] = fma(c, v_j[d], corr[d])
 *   den = (exp2(-m) + (float)(cnt - |P|) * p1) + dp
 *   y[d] = chain_r fma(sq_i[r], M_i[r][d])
 *   out[d] = fma(p1, y[d], corr[d]) * (1/den);  lse2 = m + log2(den). */
static void forward_impl(const float* sq, const float* sk, const float* v, const int32_t* iq,
                         const int32_t* ik, const uint8_t* hard, const float* lut,
                         long lut_stride, int B, long N, int H, int R, int DV, float* out,
                         float* lse2, int32_t* lmax, int32_t* jarg, int threads,
                         const int32_t* wlo, const uint8_t* dense);

void orc_forward(const float* sq, const float* sk, const float* v, const int32_t* iq,
                 const int32_t* ik, const uint8_t* hard, const float* lut, long lut_stride,
                 int B, long N, int H, int R, int DV, float* out, float* lse2, int32_t* lmax,
                 int32_t* jarg, int threads) {
    forward_impl(sq, sk, v, iq, ik, hard, lut, lut_stride, B, N, H, R, DV, out, lse2, lmax,
                 jarg, threads, NULL, NULL);
}

/* orc_forward with query resets: wlo [B*H*N] holds, per query, the last reset position at or
 * before it (0 without one); walks of that query stop there.  Bigram pairs are still every
 * key whose (previous, current) labels equal the query's; a pair cut by a reset has L = 1. */
void orc_forward_reset(const float* sq, const float* sk, const float* v, const int32_t* iq,
                       const int32_t* ik, const uint8_t* hard, const float* lut,
                       long lut_stride, int B, long N, int H, int R, int DV, float* out,
                       float* lse2, int32_t* lmax, int32_t* jarg, int threads,
                       const int32_t* wlo) {
    forward_impl(sq, sk, v, iq, ik, hard, lut, lut_stride, B, N, H, R, DV, out, lse2, lmax,
                 jarg, threads, wlo, NULL);
}

/* The forward with an explicit row classification: dense [B*H] (1: the direct definition,
 * 0: the decomposed one), or NULL for orc_dense_row's.  wlo may be NULL. */
void orc_forward_flags(const float* sq, const float* sk, const float* v, const int32_t* iq,
                       const int32_t* ik, const uint8_t* hard, const float* lut,
                       long lut_stride, int B, long N, int H, int R, int DV, float* out,
                       float* lse2, int32_t* lmax, int32_t* jarg, int threads,
                       const int32_t* wlo, const uint8_t* dense) {
    forward_impl(sq, sk, v, iq, ik, hard, lut, lut_stride, B, N, H, R, DV, out, lse2, lmax,
                 jarg, threads, wlo, dense);
}

static void forward_impl(const float* sq, const float* sk, const float* v, const int32_t* iq,
                         const int32_t* ik, const uint8_t* hard, const float* lut,
                         long lut_stride, int B, long N, int H, int R, int DV, float* out,
                         float* lse2, int32_t* lmax, int32_t* jarg, int threads,
                         const int32_t* wlo, const uint8_t* dense) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const int32_t* q = iq + (long)bh * N;
        const int32_t* k = ik + (long)bh * N;
        const float* tab = lut + (long)h * lut_stride;
        if (!hard[bh]) {
            for (long i = 0; i < N; ++i) {
                long row = ((long)b * N + i) * H + h;
                for (int d = 0; d < DV; ++d) out[row * DV + d] = 0.0f;
                lse2[(long)bh * N + i] = 0.0f;
                if (lmax) lmax[(long)bh * N + i] = 0;
                if (jarg) jarg[(long)bh * N + i] = -1;
            }
            continue;
        }
        const int mode = dense ? dense[bh] : row_mode(q, k, N, R, DV, wlo != NULL);
        Levels lv;
        if (mode == 3 && levels_build(q, k, N, &lv)) {
            const long so = (long)bh * N;
            level_forward_row(sq, sk, v, tab, b, h, N, H, R, DV, &lv, out, lse2 + so,
                              lmax ? lmax + so : NULL, jarg ? jarg + so : NULL);
            free(lv.ent);
            continue;
        }
        if (mode == 4) {
            const long so = (long)bh * N;
            prefix_forward_row(sq, sk, v, q, k, tab, b, h, N, H, R, DV, out, lse2 + so,
                               lmax ? lmax + so : NULL, jarg ? jarg + so : NULL);
            continue;
        }
        if (mode == 1 || mode == 3) {
            const long so = (long)bh * N;
            direct_forward_row(sq, sk, v, q, k, tab, b, h, N, H, R, DV, out, lse2 + so,
                               lmax ? lmax + so : NULL, jarg ? jarg + so : NULL,
                               wlo ? wlo + so : NULL);
            continue;
        }
        int32_t* qo = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
        int32_t* ko = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
        int32_t* pj = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
        int32_t* pl = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
        float* M = (float*)malloc(sizeof(float) * (size_t)R * DV);
        float* corr = (float*)malloc(sizeof(float) * (size_t)DV);
        sort_by_label(q, N, qo);
        sort_by_label(k, N, ko);
        const float lut1 = tab[1];
        long t = 0;
        while (t < N) {
            const uint32_t lbl = (uint32_t)q[qo[t]];
            long te = t;
            while (te < N && (uint32_t)q[qo[te]] == lbl) ++te;
            const long kb = label_lb(k, ko, N, lbl);
            long ke = kb;
            while (ke < N && (uint32_t)k[ko[ke]] == lbl) ++ke;
            for (long e = 0; e < (long)R * DV; ++e) M[e] = 0.0f;
            long kc = kb;
            int cnt = 0, last = -1;
            for (; t < te; ++t) {
                const long i = qo[t];
                while (kc < ke && ko[kc] <= i) {
                    const long j = ko[kc];
                    const long krow = ((long)b * N + j) * H + h;
                    for (int r = 0; r < R; ++r)
                        for (int d = 0; d < DV; ++d)
                            M[r * DV + d] = fmaf(sk[krow * R + r], v[krow * DV + d], M[r * DV + d]);
                    ++cnt;
                    last = (int)j;
                    ++kc;
                }
                const long row = ((long)b * N + i) * H + h;
                const float* sqi = sq + row * R;
                /* bigram pairs among the valid keys, ascending j */
                int np = 0;
                if (i >= 1)
                    for (long x = kb; x < kc; ++x) {
                        const long j = ko[x];
                        if (j >= 1 && k[j - 1] == q[i - 1]) {
                            pj[np] = (int32_t)j;
                            pl[np] = (int32_t)(wlo ? orc_suffix_walk_from(
                                                         q, k, i, j, wlo[(long)bh * N + i])
                                                   : orc_suffix_walk(q, k, i, j));
                            ++np;
                        }
                    }
                float m = 0.0f;
                if (cnt > 0 && lut1 > m) m = lut1;
                int32_t best = 0, bj = -1;
                for (int x = 0; x < np; ++x) {
                    if (tab[pl[x]] > m) m = tab[pl[x]];
                    if (pl[x] >= best) { best = pl[x]; bj = pj[x]; }
                }
                if (np == 0 && cnt > 0) { best = 1; bj = last; }
                const float p1 = orc_exp2f(lut1 - m);
                float dp = 0.0f;
                for (int d = 0; d < DV; ++d) corr[d] = 0.0f;
                for (int x = 0; x < np; ++x) {
                    const long krow = ((long)b * N + pj[x]) * H + h;
                    const float p = orc_exp2f(tab[pl[x]] - m);
                    dp = dp + p;
                    const float s = dot_chain(sqi, sk + krow * R, R);
                    const float c = (p - p1) * s;
                    for (int d = 0; d < DV; ++d) corr[d] = fmaf(c, v[krow * DV + d], corr[d]);
                }
                const float den = (orc_exp2f(-m) + (float)(cnt - np) * p1) + dp;
                const float rden = 1.0f / den;
                float* o = out + row * DV;
                for (int d = 0; d < DV; ++d) {
                    float y = 0.0f;
                    for (int r = 0; r < R; ++r) y = fmaf(sqi[r], M[r * DV + d], y);
                    o[d] = fmaf(p1, y, corr[d]) * rden;
                }
                lse2[(long)bh * N + i] = m + orc_log2f(den);
                if (lmax) lmax[(long)bh * N + i] = best;
                if (jarg) jarg[(long)bh * N + i] = bj;
            }
        }
        free(qo); free(ko); free(pj); free(pl); free(M); free(corr);
    }
}

/* Backward.  Per row i (l2 = lse2_i, c = G[i+1], G the dlog table):
 *   P1 = exp2(LUT[1]-l2); g1 = G[1]-c; q1 = P1*g1
 *   zq[r] = rg_reduce(dO_i, M_i[r]);  se0 = chain_r fma(sq_i[r], zq[r])
 *   for j in P (ascending): p = exp2(LUT[L]-l2); dp = p-P1; s = chain(sq_i.sk_j);
 *       e = tree(dO_i.v_j); g = G[L]-c; a = p*g - q1; de = dp*e; ds = dp*s;
 *       cdq[r] = fma(de, sk_j[r], cdq[r]); cu = fma(ds, e, cu); cvv = cvv + a;
 *       cw = fma(a, s*e, cw); cz = cz + dp
 *   dsq[r] = fma(P1, zq[r], cdq[r]); u = fma(P1, se0, cu); vv = fma(cnt, q1, cvv);
 *   w = fma(q1, se0, cw); z = fma(cnt, P1, cz)
 *   f = exp2(-l2); mass = z+f; mean = fma(-f, c, vv)/mass; rowtau = fma(-u, mean, w)/mass
 * Per key j (valid queries i >= j of the same label):
 *   N_j[r][d] = fma chain over valid queries, DESCENDING i, of (P1_i*sq_i[r]) * dO_i[d]
 *   dv0[d] = chain_r fma(sk_j[r], N[r][d]);  dsk0[r] = lane_reduce(N[r], v_j)
 *   for bigram queries i of j (ascending i): p = exp2(LUT[L]-l2_i); dp = p - P1_i;
 *       s = chain(sq_i.sk_j); e = tree(dO_i.v_j); cdk[r] = fma(dp*e, sq_i[r], cdk[r]);
 *       cdv[d] = fma(dp*s, dO_i[d], cdv[d])
 *   dsk[r] = dsk0[r] + cdk[r];  dv[d] = dv0[d] + cdv[d]  (only for keys with bigram pairs). */
void orc_backward_flags(const float* sq, const float* sk, const float* v, const float* dout,
                        const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                        const float* lut, const float* dlut, long lut_stride,
                        const float* lse2in, int B, long N, int H, int R, int DV, float* dsq,
                        float* dsk, float* dv, float* rowtau, int threads,
                        const uint8_t* dense);

void orc_backward(const float* sq, const float* sk, const float* v, const float* dout,
                  const int32_t* iq, const int32_t* ik, const uint8_t* hard, const float* lut,
                  const float* dlut, long lut_stride, const float* lse2in, int B, long N, int H,
                  int R, int DV, float* dsq, float* dsk, float* dv, float* rowtau, int threads) {
    orc_backward_flags(sq, sk, v, dout, iq, ik, hard, lut, dlut, lut_stride, lse2in, B, N, H,
                       R, DV, dsq, dsk, dv, rowtau, threads, NULL);
}

/* The backward with an explicit row classification (dense as in orc_forward_flags). */
void orc_backward_flags(const float* sq, const float* sk, const float* v, const float* dout,
                        const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                        const float* lut, const float* dlut, long lut_stride,
                        const float* lse2in, int B, long N, int H, int R, int DV, float* dsq,
                        float* dsk, float* dv, float* rowtau, int threads,
                        const uint8_t* dense) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (int bh = 0; bh < B * H; ++bh) {
        const int b = bh / H, h = bh % H;
        const int32_t* q = iq + (long)bh * N;
        const int32_t* k = ik + (long)bh * N;
        const float* tab = lut + (long)h * lut_stride;
        const float* gt = dlut + (long)h * lut_stride;
        const float* l2v = lse2in + (long)bh * N;
        for (long x = 0; x < N; ++x) {
            long row = ((long)b * N + x) * H + h;
            for (int r = 0; r < R; ++r) { dsq[row * R + r] = 0.0f; dsk[row * R + r] = 0.0f; }
            for (int d = 0; d < DV; ++d) dv[row * DV + d] = 0.0f;
            rowtau[(long)bh * N + x] = 0.0f;
        }
        if (!hard[bh]) continue;
        const int mode = dense ? dense[bh] : row_mode(q, k, N, R, DV, 0);
        Levels lv;
        if (mode == 3 && levels_build(q, k, N, &lv)) {
            level_backward_row(sq, sk, v, dout, tab, gt, l2v, b, h, N, H, R, DV, &lv, dsq, dsk,
                               dv, rowtau + (long)bh * N);
            free(lv.ent);
            continue;
        }
        if (mode == 4) {
            prefix_backward_row(sq, sk, v, dout, q, k, tab, gt, l2v, b, h, N, H, R, DV, dsq,
                                dsk, dv, rowtau + (long)bh * N);
            continue;
        }
        if (mode == 1 || mode == 3) {
            direct_backward_row(sq, sk, v, dout, q, k, tab, gt, l2v, b, h, N, H, R, DV, dsq,
                                dsk, dv, rowtau + (long)bh * N);
            continue;
        }
        int32_t* qo = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
        int32_t* ko = (int32_t*)malloc(sizeof(int32_t) * (size_t)N);
        float* M = (float*)malloc(sizeof(float) * (size_t)R * DV);
        float* zq = (float*)malloc(sizeof(float) * (size_t)R);
        float* cd = (float*)malloc(sizeof(float) * (size_t)(R + DV));
        float* a = (float*)malloc(sizeof(float) * (size_t)R);
        sort_by_label(q, N, qo);
        sort_by_label(k, N, ko);
        const float lut1 = tab[1];
        /* ---- rows */
        long t = 0;
        while (t < N) {
            const uint32_t lbl = (uint32_t)q[qo[t]];
            long te = t;
            while (te < N && (uint32_t)q[qo[te]] == lbl) ++te;
            const long kb = label_lb(k, ko, N, lbl);
            long ke = kb;
            while (ke < N && (uint32_t)k[ko[ke]] == lbl) ++ke;
            for (long e = 0; e < (long)R * DV; ++e) M[e] = 0.0f;
            long kc = kb;
            int cnt = 0;
            for (; t < te; ++t) {
                const long i = qo[t];
                while (kc < ke && ko[kc] <= i) {
                    const long krow = ((long)b * N + ko[kc]) * H + h;
                    for (int r = 0; r < R; ++r)
                        for (int d = 0; d < DV; ++d)
                            M[r * DV + d] = fmaf(sk[krow * R + r], v[krow * DV + d], M[r * DV + d]);
                    ++cnt;
                    ++kc;
                }
                const long row = ((long)b * N + i) * H + h;
                const float* sqi = sq + row * R;
                const float* doi = dout + row * DV;
                const float l2 = l2v[i];
                const float c = gt[i + 1];
                const float P1 = orc_exp2f(lut1 - l2);
                const float g1 = gt[1] - c;
                const float q1 = P1 * g1;
                for (int r = 0; r < R; ++r) zq[r] = rg_reduce(doi, M + (long)r * DV, DV, R);
                const float se0 = dot_chain(sqi, zq, R);
                float cu = 0.0f, cvv = 0.0f, cw = 0.0f, cz = 0.0f;
                for (int r = 0; r < R; ++r) cd[r] = 0.0f;
                if (i >= 1)
                    for (long x = kb; x < kc; ++x) {
                        const long j = ko[x];
                        if (!(j >= 1 && k[j - 1] == q[i - 1])) continue;
                        const long L = orc_suffix_walk(q, k, i, j);
                        const long krow = ((long)b * N + j) * H + h;
                        const float* skj = sk + krow * R;
                        const float p = orc_exp2f(tab[L] - l2);
                        const float dp = p - P1;
                        const float s = dot_chain(sqi, skj, R);
                        const float e = tree_dot(doi, v + krow * DV, DV);
                        const float g = gt[L] - c;
                        const float av = p * g - q1;
                        const float de = dp * e, ds = dp * s;
                        for (int r = 0; r < R; ++r) cd[r] = fmaf(de, skj[r], cd[r]);
                        cu = fmaf(ds, e, cu);
                        cvv = cvv + av;
                        cw = fmaf(av, s * e, cw);
                        cz = cz + dp;
                    }
                for (int r = 0; r < R; ++r) dsq[row * R + r] = fmaf(P1, zq[r], cd[r]);
                const float fc = (float)cnt;
                const float u = fmaf(P1, se0, cu);
                const float vv = fmaf(fc, q1, cvv);
                const float w = fmaf(q1, se0, cw);
                const float z = fmaf(fc, P1, cz);
                const float f = orc_exp2f(-l2);
                const float mass = z + f;
                const float mean = fmaf(-f, c, vv) / mass;
                rowtau[(long)bh * N + i] = fmaf(-u, mean, w) / mass;
            }
        }
        /* ---- keys: descending merge per label */
        long tk = N - 1;
        while (tk >= 0) {
            const uint32_t lbl = (uint32_t)k[ko[tk]];
            long tb = tk;
            while (tb >= 0 && (uint32_t)k[ko[tb]] == lbl) --tb;
            /* queries of this label: [qb, qe) in label order */
            const long qb = label_lb(q, qo, N, lbl);
            long qe = qb;
            while (qe < N && (uint32_t)q[qo[qe]] == lbl) ++qe;
            for (long e = 0; e < (long)R * DV; ++e) M[e] = 0.0f; /* N matrix */
            long qc = qe - 1;
            for (; tk > tb; --tk) {
                const long j = ko[tk];
                while (qc >= qb && qo[qc] >= j) {
                    const long i = qo[qc];
                    const long row = ((long)b * N + i) * H + h;
                    const float P1 = orc_exp2f(lut1 - l2v[i]);
                    for (int r = 0; r < R; ++r) a[r] = P1 * sq[row * R + r];
                    for (int r = 0; r < R; ++r)
                        for (int d = 0; d < DV; ++d)
                            M[r * DV + d] = fmaf(a[r], dout[row * DV + d], M[r * DV + d]);
                    --qc;
                }
                const long krow = ((long)b * N + j) * H + h;
                const float* skj = sk + krow * R;
                const float* vj = v + krow * DV;
                for (int r = 0; r < R + DV; ++r) cd[r] = 0.0f;
                int npair = 0;
                if (j >= 1)
                    for (long x = qc + 1; x < qe; ++x) {
                        const long i = qo[x];
                        if (!(i >= 1 && q[i - 1] == k[j - 1])) continue;
                        const long L = orc_suffix_walk(q, k, i, j);
                        const long row = ((long)b * N + i) * H + h;
                        const float* sqi = sq + row * R;
                        const float* doi = dout + row * DV;
                        const float l2 = l2v[i];
                        const float P1 = orc_exp2f(lut1 - l2);
                        const float p = orc_exp2f(tab[L] - l2);
                        const float dp = p - P1;
                        const float s = dot_chain(sqi, skj, R);
                        const float e = tree_dot(doi, vj, DV);
                        const float de = dp * e, ds = dp * s;
                        for (int r = 0; r < R; ++r) cd[r] = fmaf(de, sqi[r], cd[r]);
                        for (int d = 0; d < DV; ++d) cd[R + d] = fmaf(ds, doi[d], cd[R + d]);
                        ++npair;
                    }
                /* corrections are added only to keys that have bigram pairs */
                for (int r = 0; r < R; ++r) {
                    const float base = lane_reduce(M + (long)r * DV, vj, DV, R);
                    dsk[krow * R + r] = npair ? base + cd[r] : base;
                }
                for (int d = 0; d < DV; ++d) {
                    float y = 0.0f;
                    for (int r = 0; r < R; ++r) y = fmaf(skj[r], M[r * DV + d], y);
                    dv[krow * DV + d] = npair ? y + cd[R + d] : y;
                }
            }
        }
        free(qo); free(ko); free(M); free(zq); free(cd); free(a);
    }
}

/* ---------------- vocabulary labels ----------------
 * labels[b,h,n] = argmax_v sum_d x[b,n,h,d] * vocab[h*vhs + v*D + d], summed in d order in
 * double, first index on ties -- the argmax of
 * dism_v3/python/flash_dism/reference/dism_v3_ref.py:159-162 (torch argmax returns the first
 * maximal index).  The products of bf16 values are exact in double; the sum is exact while the
 * products' exponents span less than about 53 - 16 - log2(D) bits (not for arbitrarily spread
 * inputs, e.g. mixing subnormals with large values).  tests/test_oracle.py checks it against
 * exact rational arithmetic on random rows, exact ties and one-ulp near ties. */
void orc_vocab_labels(const float* x, const float* vocab, long vhs, int B, long N, int H, long V,
                      int D, int32_t* labels) {
    for (int b = 0; b < B; ++b)
        for (long n = 0; n < N; ++n)
            for (int h = 0; h < H; ++h) {
                const float* xt = x + (((long)b * N + n) * H + h) * D;
                double best = -INFINITY;
                long bi = 0;
                for (long v = 0; v < V; ++v) {
                    const float* e = vocab + (long)h * vhs + v * D;
                    double s = 0.0;
                    for (int d = 0; d < D; ++d) s += (double)xt[d] * (double)e[d];
                    if (s > best) { best = s; bi = v; }
                }
                labels[((long)b * H + h) * N + n] = (int32_t)bi;
            }
}
