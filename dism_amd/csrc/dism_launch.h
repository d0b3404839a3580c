// dism_launch.h -- host-side launchers exported by the .hip translation units to the C-ABI
// layer (dism_capi.cpp).  Plain pointers and sizes only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dism {

enum { DTYPE_BF16 = 0, DTYPE_F32 = 1 };
constexpr int BUCKETS = 256;          // symbol buckets (label & 255)
constexpr int CHUNK = 64;             // owners per wave

// Label buckets of one call (see dism_bucket.hip).  [BH*N] positions, [BH*(BUCKETS+1)] tables.
struct BucketArgs {
    const int32_t* iq;
    const int32_t* ik;
    long BH;
    int n;
    int32_t* qpos;
    int32_t* kpos;
    int32_t* qoff;
    int32_t* koff;
    int32_t* qcs;
    int32_t* kcs;
};

// Everything the sweep kernels share.
struct SweepCommon {
    int B, H, n;
    const int32_t* iq;     // [B,H,N]
    const int32_t* ik;     // [B,H,N]
    const uint8_t* hard;   // [B*H] sequence flags
    const int32_t* bound;  // composed boundary [B,H,(N-1)/strip,N] or null
    int strip;
    const float* lut;      // [H, lut_stride] log2 weights
    long lut_stride;
    const int32_t* qpos;   // buckets (dism_bucket.hip)
    const int32_t* kpos;
    const int32_t* qoff;
    const int32_t* koff;
    const int32_t* qcs;
    const int32_t* kcs;
    const int32_t* bad;    // [B*H] non-finite input flags (masked accumulation when set)
    int slots;             // chunk slots per (b,h): ceil(N/64) + BUCKETS
    const uint32_t* prec;  // partner records in bucket order, [B*H*N][pstride] words
    int pstride;
};

// Partner records (dism_bucket.hip): for each (b,h) and bucket-sorted index t of one side,
//   word 0: position p, 1: label[p], 2: label[p-1] (0 at p = 0), 3: extra (lse2[p] bits for
//   query records, 0 for key records), then the readout row (R elements of T) and the value
//   row (DV elements of T) as raw 32-bit words; stride rounded up to 4 words.
struct RecordArgs {
    int B, H, n;
    const int32_t* pos;    // [B*H*N] bucket-sorted positions of the side
    const int32_t* lab;    // [B,H,N] labels of the side
    const void* rrow;      // [B,N,H,R] readout rows (sk for keys, sq for queries)
    const void* vrow;      // [B,N,H,DV] value rows (v for keys, dO for queries)
    const float* extra;    // [B,H,N] or null
    int rw, vw, stride;    // words of readout row, value row, record stride
    int dtype;             // element type of the rows (non-finite check)
    uint32_t* rec;
    int32_t* bad;          // [B*H] raised when a copied row holds a non-finite value
};

struct ForwardArgs {
    SweepCommon c;
    const void* sq;        // [B,N,H,R]  bf16|f32
    const void* sk;        // [B,N,H,R]
    const void* v;         // [B,N,H,DV]
    void* out;             // [B,N,H,DV] bf16 (out_dtype 0) or f32 (1)
    int out_dtype;
    float* lse2;           // [B,H,N]
    int32_t* lmax;         // [B,H,N] longest match length (nullable)
    int32_t* jarg;         // [B,H,N] key of the longest match, ties -> latest (nullable)
};

struct BackwardArgs {
    SweepCommon c;
    const void* sq;
    const void* sk;
    const void* v;
    const void* dout;      // [B,N,H,DV]
    const float* dlut;     // [H, lut_stride] natural-tau derivative of ln W_L
    const float* lse2;     // [B,H,N] saved log2 normalizer
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
hipError_t launch_fill_i32(int32_t* p, long count, int32_t value, hipStream_t s);
hipError_t launch_buckets(const BucketArgs& a, hipStream_t s);
hipError_t launch_records(const RecordArgs& a, hipStream_t s);
hipError_t launch_nonfinite(const void* x, int dtype, long B, long N, long H, int D,
                            int32_t* flags, hipStream_t s);
// return hipErrorInvalidValue for an unsupported (R, DV, dtype)
hipError_t launch_forward(const ForwardArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_backward_rows(const BackwardArgs& a, int R, int DV, int dtype, hipStream_t s);
hipError_t launch_backward_keys(const BackwardArgs& a, int R, int DV, int dtype, hipStream_t s);

}  // namespace dism
