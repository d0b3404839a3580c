// dism_launch.h -- host-side launchers exported by the .hip translation units to the C-ABI
// layer (dism_capi.cpp).  Plain pointers and sizes only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dism {

enum { DTYPE_BF16 = 0, DTYPE_F32 = 1 };

// Forward sweep arguments (one (b,h) row = one batch-head pair of length n).
struct ForwardArgs {
    const void* sq;        // [B,N,H,R]  bf16|f32
    const void* sk;        // [B,N,H,R]
    const void* v;         // [B,N,H,DV]
    const int32_t* iq;     // [B,H,N]
    const int32_t* ik;     // [B,H,N]
    const uint8_t* hard;   // [B*H] sequence flags
    const int32_t* bound;  // composed boundary [B,H,(N-1)/strip,N] or null
    int strip;
    const float* lut;      // [H, lut_stride] log2 weights
    long lut_stride;
    int B, H, n;
    void* out;             // [B,N,H,DV] bf16 (out_dtype 0) or f32 (1)
    int out_dtype;
    float* lse2;           // [B,H,N]
    int32_t* lmax;         // [B,H,N] longest match length (nullable)
    int32_t* jarg;         // [B,H,N] key of the longest match, ties -> latest (nullable)
};

struct BackwardArgs {
    const void* sq;
    const void* sk;
    const void* v;
    const void* dout;      // [B,N,H,DV]
    const int32_t* iq;
    const int32_t* ik;
    const uint8_t* hard;
    const int32_t* bound;
    int strip;
    const float* lut;
    const float* dlut;     // [H, lut_stride] natural-tau derivative of ln W_L
    long lut_stride;
    const float* lse2;     // [B,H,N] saved log2 normalizer
    int B, H, n;
    float* dsq;            // [B,N,H,R] fp32
    float* dsk;            // [B,N,H,R] fp32
    float* dv;             // [B,N,H,DV] fp32
    float* rowtau;         // [B,H,N] fp32 per-row tau gradient terms
};

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
// returns hipErrorInvalidValue for an unsupported (R, DV, dtype)
hipError_t launch_forward(const ForwardArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_backward_rows(const BackwardArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_backward_keys(const BackwardArgs& a, int R, int DV, int dtype, hipStream_t s);

}  // namespace dism
