// dism_capi.cpp -- extern "C" boundary of libdism_hip.so: argument validation, launch
// dispatch, thread-local error text.  Declarations and reference mapping: include/dism_hard.h.
#include <hip/hip_runtime.h>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/dism_hard.h"
#include "dism_launch.h"

namespace {
thread_local std::string g_error;

int32_t fail(int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int32_t ok() {
    g_error.clear();
    return DISM_OK;
}

int32_t hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return ok();
    if (e == hipErrorInvalidValue)
        return fail(DISM_ERR_UNSUPPORTED, "%s: unsupported readout/value dims or dtype", what);
    return fail(DISM_ERR_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

bool dims_ok(int64_t B, int64_t N, int64_t H) {
    return B > 0 && H > 0 && N > 0 && N <= INT_MAX - 1024 && B * H <= INT_MAX &&
           ((N + 255) / 256) * B * H <= INT_MAX;
}
bool rdv_ok(int32_t R, int32_t DV) {
    return (R == 2 || R == 4 || R == 8 || R == 16 || R == 32) && (DV == 32 || DV == 64 || DV == 128);
}
hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
}  // namespace

extern "C" {

const char* dism_last_error(void) { return g_error.c_str(); }
int32_t dism_abi_version(void) { return 1; }

int32_t dism_sign_labels(const void* x, int32_t dtype, int64_t B, int64_t N, int64_t H, int32_t d,
                         int32_t* labels, void* stream) {
    if (!x || !labels) return fail(DISM_ERR_INVALID, "sign labels: null pointer");
    if (!dims_ok(B, N, H)) return fail(DISM_ERR_INVALID, "sign labels: positive dimensions required");
    if (d < 1 || d > 30) return fail(DISM_ERR_INVALID, "sign labels: symbol width must be in [1,30]");
    if (dtype != DISM_BF16 && dtype != DISM_F32)
        return fail(DISM_ERR_UNSUPPORTED, "sign labels: dtype must be bf16 or f32");
    return hip_status(dism::launch_sign_labels(x, dtype, B, N, H, d, labels, S(stream)), "sign labels");
}

int32_t dism_hard_log_weights(const float* tau, int32_t H, int64_t max_length, float* lut,
                              void* stream) {
    if (!tau || !lut) return fail(DISM_ERR_INVALID, "tau must be contiguous FP32 [H]");
    if (H <= 0 || H > 65535) return fail(DISM_ERR_INVALID, "tau must be contiguous FP32 [H]");
    if (max_length <= 0 || max_length > INT_MAX - 1024)
        return fail(DISM_ERR_INVALID, "LUT maximum length must be positive");
    return hip_status(dism::launch_log_weights(tau, H, max_length + 1, lut, S(stream)),
                      "hard log weights");
}

int32_t dism_hard_dlog_weights(const float* tau, int32_t H, int64_t stride, float* dlut,
                               void* stream) {
    if (!tau || !dlut) return fail(DISM_ERR_INVALID, "tau must be contiguous FP32 [H]");
    if (H <= 0 || H > 65535 || stride <= 0 || stride > INT_MAX)
        return fail(DISM_ERR_INVALID, "invalid derivative table shape");
    return hip_status(dism::launch_dlog_weights(tau, H, stride, dlut, S(stream)),
                      "hard dlog weights");
}

int32_t dism_hard_summary(const int32_t* iq, const int32_t* ik, const uint8_t* hard, int64_t B,
                          int64_t H, int64_t N, int32_t* summary, void* stream) {
    if (!iq || !ik || !hard || !summary) return fail(DISM_ERR_INVALID, "hard summary: null pointer");
    if (!dims_ok(B, N, H)) return fail(DISM_ERR_INVALID, "positive dimensions required");
    if ((N - 1) / 32 == 0) return ok();
    return hip_status(dism::launch_boundary(iq, ik, hard, B * H, (int)N, 32, 0, 1, summary,
                                            S(stream)), "hard summary");
}

int32_t dism_hard_chunk(const int32_t* summary, int32_t* boundary, int64_t BH, int64_t N,
                        void* stream) {
    if (!summary || !boundary) return fail(DISM_ERR_INVALID, "hard chunk: null pointer");
    if (BH <= 0 || BH > 65535 || N <= 0 || N > INT_MAX - 1024)
        return fail(DISM_ERR_INVALID, "invalid fixed batch/head count");
    int64_t C = (N - 1) / 32;
    if (C == 0) return ok();
    return hip_status(dism::launch_chunk(summary, boundary, BH, C, (int)N, S(stream)), "hard chunk");
}

int32_t dism_hard_boundary(const int32_t* iq, const int32_t* ik, const uint8_t* hard, int64_t B,
                           int64_t H, int64_t N, int32_t strip, int32_t fill_all,
                           int32_t* boundary, void* stream) {
    if (!iq || !ik || !hard || !boundary) return fail(DISM_ERR_INVALID, "hard boundary: null pointer");
    if (!dims_ok(B, N, H)) return fail(DISM_ERR_INVALID, "positive dimensions required");
    if (strip < 1) return fail(DISM_ERR_INVALID, "boundary strip height must be positive");
    if ((N - 1) / strip == 0) return ok();
    if (B * H > 65535) return fail(DISM_ERR_INVALID, "hard boundary: too many batch-head rows");
    return hip_status(dism::launch_boundary(iq, ik, hard, B * H, (int)N, strip, 1, fill_all,
                                            boundary, S(stream)), "hard boundary");
}

int32_t dism_hard_readout(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                          const int32_t* boundary, int32_t strip, const float* lut,
                          int64_t lut_stride, int64_t B, int64_t N, int64_t H, int32_t R,
                          int32_t DV, void* out, int32_t out_dtype, float* lse2, int32_t* lmax,
                          int32_t* jarg, void* stream) {
    if (!sq || !sk || !v || !iq || !ik || !hard || !lut || !out || !lse2)
        return fail(DISM_ERR_INVALID, "hard readout: null pointer");
    if (!dims_ok(B, N, H)) return fail(DISM_ERR_INVALID, "positive dimensions required");
    if (!rdv_ok(R, DV))
        return fail(DISM_ERR_UNSUPPORTED, "hard readout: unsupported R=%d DV=%d", R, DV);
    if (dtype != DISM_BF16 && dtype != DISM_F32)
        return fail(DISM_ERR_UNSUPPORTED, "hard readout: vector dtype must be bf16 or f32");
    if (out_dtype != DISM_BF16 && out_dtype != DISM_F32)
        return fail(DISM_ERR_UNSUPPORTED, "hard readout: output dtype must be bf16 or f32");
    if (lut_stride < N + 1) return fail(DISM_ERR_INVALID, "hard log-weight table is too short");
    if (boundary && strip < 1) return fail(DISM_ERR_INVALID, "invalid hard boundary strip");
    dism::ForwardArgs a{sq, sk, v, iq, ik, hard, boundary, boundary ? strip : 0, lut, lut_stride,
                        (int)B, (int)H, (int)N, out, out_dtype, lse2, lmax, jarg};
    return hip_status(dism::launch_forward(a, R, DV, dtype, S(stream)), "hard readout");
}

static int32_t backward_args(const void* sq, const void* sk, const void* v, const void* dout,
                             int32_t dtype, const int32_t* iq, const int32_t* ik,
                             const uint8_t* hard, const int32_t* boundary, int32_t strip,
                             const float* lut, const float* dlut, int64_t lut_stride,
                             const float* lse2, int64_t B, int64_t N, int64_t H, int32_t R,
                             int32_t DV, float* dsq, float* dsk, float* dv, float* rowtau,
                             bool need_rows, bool need_keys, dism::BackwardArgs* a) {
    if (!sq || !sk || !v || !dout || !iq || !ik || !hard || !lut || !lse2)
        return fail(DISM_ERR_INVALID, "hard backward: null pointer");
    if ((need_rows && (!dlut || !dsq || !rowtau)) || (need_keys && (!dsk || !dv)))
        return fail(DISM_ERR_INVALID, "hard backward: null pointer");
    if (!dims_ok(B, N, H)) return fail(DISM_ERR_INVALID, "positive dimensions required");
    if (!rdv_ok(R, DV))
        return fail(DISM_ERR_UNSUPPORTED, "hard backward: unsupported R=%d DV=%d", R, DV);
    if (dtype != DISM_BF16 && dtype != DISM_F32)
        return fail(DISM_ERR_UNSUPPORTED, "hard backward: vector dtype must be bf16 or f32");
    if (lut_stride < N + 1) return fail(DISM_ERR_INVALID, "hard log-weight table is too short");
    if (boundary && strip < 1) return fail(DISM_ERR_INVALID, "invalid hard boundary strip");
    *a = dism::BackwardArgs{sq, sk, v, dout, iq, ik, hard, boundary, boundary ? strip : 0, lut,
                            dlut, lut_stride, lse2, (int)B, (int)H, (int)N, dsq, dsk, dv, rowtau};
    return DISM_OK;
}

int32_t dism_hard_backward_queries(const void* sq, const void* sk, const void* v,
                                   const void* dout, int32_t dtype, const int32_t* iq,
                                   const int32_t* ik, const uint8_t* hard,
                                   const int32_t* boundary, int32_t strip, const float* lut,
                                   const float* dlut, int64_t lut_stride, const float* lse2,
                                   int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                   float* dsq, float* rowtau, void* stream) {
    dism::BackwardArgs a;
    int32_t st = backward_args(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip, lut, dlut,
                               lut_stride, lse2, B, N, H, R, DV, dsq, nullptr, nullptr, rowtau,
                               true, false, &a);
    if (st) return st;
    return hip_status(dism::launch_backward_rows(a, R, DV, dtype, S(stream)), "hard backward rows");
}

int32_t dism_hard_backward_keys(const void* sq, const void* sk, const void* v, const void* dout,
                                int32_t dtype, const int32_t* iq, const int32_t* ik,
                                const uint8_t* hard, const int32_t* boundary, int32_t strip,
                                const float* lut, int64_t lut_stride, const float* lse2,
                                int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                float* dsk, float* dv, void* stream) {
    dism::BackwardArgs a;
    int32_t st = backward_args(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip, lut,
                               nullptr, lut_stride, lse2, B, N, H, R, DV, nullptr, dsk, dv,
                               nullptr, false, true, &a);
    if (st) return st;
    return hip_status(dism::launch_backward_keys(a, R, DV, dtype, S(stream)), "hard backward keys");
}

int32_t dism_hard_tau_reduce(const float* rowtau, int64_t B, int64_t H, int64_t N, float* dtau,
                             void* stream) {
    if (!rowtau || !dtau) return fail(DISM_ERR_INVALID, "tau reduce: null pointer");
    if (!dims_ok(B, N, H)) return fail(DISM_ERR_INVALID, "positive dimensions required");
    return hip_status(dism::launch_tau_reduce(rowtau, (int)B, (int)H, N, dtau, S(stream)),
                      "hard tau reduce");
}

int32_t dism_hard_backward(const void* sq, const void* sk, const void* v, const void* dout,
                           int32_t dtype, const int32_t* iq, const int32_t* ik,
                           const uint8_t* hard, const int32_t* boundary, int32_t strip,
                           const float* lut, const float* dlut, int64_t lut_stride,
                           const float* lse2, int64_t B, int64_t N, int64_t H, int32_t R,
                           int32_t DV, float* dsq, float* dsk, float* dv, float* rowtau,
                           float* dtau, void* stream) {
    if (!dtau) return fail(DISM_ERR_INVALID, "hard backward: null pointer");
    int32_t st = dism_hard_backward_queries(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip,
                                            lut, dlut, lut_stride, lse2, B, N, H, R, DV, dsq,
                                            rowtau, stream);
    if (st) return st;
    st = dism_hard_backward_keys(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip, lut,
                                 lut_stride, lse2, B, N, H, R, DV, dsk, dv, stream);
    if (st) return st;
    return dism_hard_tau_reduce(rowtau, B, H, N, dtau, stream);
}

}  // extern "C"
