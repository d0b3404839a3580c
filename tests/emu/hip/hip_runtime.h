// CPU emulation of the HIP subset the hard-core kernels use -- test infrastructure only
// (tests/test_emulated_kernels.py builds dism_amd/csrc with it into a separate CPU library;
// the product library never includes this file).
// Lanes are fibers.  The kernel units are compiled with -fsanitize-coverage=trace-pc, so every
// lane stops at every basic block; per wave, the lanes at the lowest code position (call stack
// compared outermost frame first) run one block at a time: lockstep execution with
// reconvergence after structured branches, as a wave64 SIMD runs it.  Wave operations
// (ballot, shuffles, readlane, DPP, permlane swaps) resolve over the lanes that execute them
// together; __syncthreads releases when every live lane has reached it.  Global memory is
// host memory (AddressSanitizer checks every access), LDS is one static copy per kernel.
#pragma once
#include <cstdint>
#include <cstring>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <tuple>
#include <utility>
#include <type_traits>
#include <array>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static
#define __align__(n) alignas(n)

struct dim3 {
    unsigned x, y, z;
    constexpr dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct alignas(16) uint4 { unsigned x, y, z, w; };
struct alignas(16) int4 { int x, y, z, w; };
struct alignas(16) float4 { float x, y, z, w; };
struct alignas(8) uint2 { unsigned x, y; };
struct alignas(8) int2 { int x, y; };
struct alignas(8) float2 { float x, y; };
inline int4 make_int4(int a, int b, int c, int d) { return int4{a, b, c, d}; }
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }
inline float2 make_float2(float a, float b) { return float2{a, b}; }
inline uint2 make_uint2(unsigned a, unsigned b) { return uint2{a, b}; }

typedef int hipError_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorUnknown = 999 };
typedef struct emu_stream* hipStream_t;
typedef struct emu_event* hipEvent_t;
enum { hipStreamNonBlocking = 1, hipEventDisableTiming = 2 };
enum hipMemcpyKind { hipMemcpyDeviceToDevice = 3 };

namespace emu {
struct Lane;
Lane* cur();
extern dim3 g_block_idx, g_grid_dim, g_block_dim;
const dim3& tid_of(Lane*);
extern hipError_t g_last_error;
void run_grid(void (*body)(void*), void* ctx, dim3 grid, dim3 block);

// wave operations (implemented in emu.cpp)
uint64_t wave_op(int kind, uint64_t value, int arg);  // returns this lane's result
enum { OP_BALLOT = 1, OP_SHFL, OP_XOR, OP_UP, OP_DOWN, OP_FIRST, OP_READLANE, OP_BARRIER,
       OP_DPP, OP_PL16A, OP_PL16B, OP_PL32A, OP_PL32B, OP_SYNC };
int lane_of_cur();

template <typename T>
inline uint64_t bits(T v) { uint64_t u = 0; std::memcpy(&u, &v, sizeof(T)); return u; }
template <typename T>
inline T unbits(uint64_t u) { T v; std::memcpy(&v, &u, sizeof(T)); return v; }

template <typename K, typename Tup, size_t... I>
inline void call_kernel(K k, Tup& t, std::index_sequence<I...>) { k(std::get<I>(t)...); }

template <typename... P, typename... A>
inline void launch(void (*k)(P...), dim3 g, dim3 b, A&&... args) {
    using Tup = std::tuple<std::decay_t<P>...>;
    struct Ctx { void (*k)(P...); Tup t; };
    Ctx* c = new Ctx{k, Tup(std::forward<A>(args)...)};
    run_grid([](void* p) {
        Ctx* cc = static_cast<Ctx*>(p);
        Tup copy = cc->t;  // by-value parameters: every lane its own copy
        call_kernel(cc->k, copy, std::index_sequence_for<P...>{});
    }, c, g, b);
    delete c;
}
}  // namespace emu

#define threadIdx (emu::tid_of(emu::cur()))
#define blockIdx (emu::g_block_idx)
#define gridDim (emu::g_grid_dim)
#define blockDim (emu::g_block_dim)

#define hipLaunchKernelGGL(k, g, b, sh, st, ...) emu::launch(k, dim3(g), dim3(b), ##__VA_ARGS__)

inline void __syncthreads() { emu::wave_op(emu::OP_SYNC, 0, 0); }
inline int __syncthreads_or(int p) { return (int)emu::wave_op(emu::OP_SYNC, p ? 1 : 0, 1); }
inline int __syncthreads_and(int p) { return (int)emu::wave_op(emu::OP_SYNC, p ? 1 : 0, 2); }
inline int __syncthreads_count(int p) { return (int)emu::wave_op(emu::OP_SYNC, p ? 1 : 0, 3); }
inline void __threadfence() {}
#define __builtin_amdgcn_fence(...) ((void)0)
#define __builtin_amdgcn_s_waitcnt(x) ((void)0)
#define __builtin_amdgcn_wave_barrier() ((void)emu::wave_op(emu::OP_BARRIER, 0, 0))

inline unsigned long long __ballot(int p) { return emu::wave_op(emu::OP_BALLOT, p ? 1 : 0, 0); }
template <typename T>
inline T __shfl(T v, int src, int width = 64) {
    (void)width;
    return emu::unbits<T>(emu::wave_op(emu::OP_SHFL, emu::bits(v), src));
}
template <typename T>
inline T __shfl_xor(T v, int m, int width = 64) {
    (void)width;
    return emu::unbits<T>(emu::wave_op(emu::OP_XOR, emu::bits(v), m));
}
template <typename T>
inline T __shfl_up(T v, unsigned d, int width = 64) {
    return emu::unbits<T>(emu::wave_op(emu::OP_UP, emu::bits(v), (int)d | (width << 8)));
}
template <typename T>
inline T __shfl_down(T v, unsigned d, int width = 64) {
    return emu::unbits<T>(emu::wave_op(emu::OP_DOWN, emu::bits(v), (int)d | (width << 8)));
}
template <typename T>
inline T emu_readfirstlane(T v) { return emu::unbits<T>(emu::wave_op(emu::OP_FIRST, emu::bits(v), 0)); }
template <typename T>
inline T emu_readlane(T v, int l) { return emu::unbits<T>(emu::wave_op(emu::OP_READLANE, emu::bits(v), l)); }
#define __builtin_amdgcn_readfirstlane(v) emu_readfirstlane(v)
#define __builtin_amdgcn_readlane(v, l) emu_readlane(v, l)
inline int emu_update_dpp(int old, int src, int ctrl, int rm, int bm, bool bc) {
    (void)old; (void)rm; (void)bm; (void)bc;
    return (int)(uint32_t)emu::wave_op(emu::OP_DPP, (uint32_t)src, ctrl);
}
#define __builtin_amdgcn_update_dpp(o, s, c, rm, bm, bc) emu_update_dpp(o, s, c, rm, bm, bc)
inline std::array<uint32_t, 2> emu_pl16(uint32_t a, uint32_t b) {
    const uint32_t r0 = (uint32_t)emu::wave_op(emu::OP_PL16A, ((uint64_t)b << 32) | a, 0);
    const uint32_t r1 = (uint32_t)emu::wave_op(emu::OP_PL16B, ((uint64_t)b << 32) | a, 0);
    return {r0, r1};
}
inline std::array<uint32_t, 2> emu_pl32(uint32_t a, uint32_t b) {
    const uint32_t r0 = (uint32_t)emu::wave_op(emu::OP_PL32A, ((uint64_t)b << 32) | a, 0);
    const uint32_t r1 = (uint32_t)emu::wave_op(emu::OP_PL32B, ((uint64_t)b << 32) | a, 0);
    return {r0, r1};
}
#define __builtin_amdgcn_permlane16_swap(a, b, fi, bc) emu_pl16(a, b)
#define __builtin_amdgcn_permlane32_swap(a, b, fi, bc) emu_pl32(a, b)
inline void emu_global_load_lds(const void* src, void* dst, int size, int, int) {
    std::memcpy(static_cast<unsigned char*>(dst) + emu::lane_of_cur() * size, src, size);
}
#define __builtin_amdgcn_global_load_lds(s, d, sz, o, a) emu_global_load_lds(s, (void*)(d), sz, o, a)
// v_mfma_f32_32x32x8_bf16 (1k): A 32x8 (lane l: row l % 32, k = 4 (l / 32) + 0..3), B 8x32
// (lane l: column l % 32, same k), C/D 32x32 (lane l: column l % 32; register r: row
// 8 (r / 4) + 4 (l / 32) + r % 4).  The wave's operands meet in a staging table at a wave
// barrier; each lane then forms its own column (products exact in fp32, summed in k order,
// added to C).  Only the vocabulary kernels use it (clang units: ext_vector_type operands).
inline float __uint_as_float(uint32_t u);
namespace emu {
struct MfmaStage { uint16_t a[64][4], b[64][4]; };
MfmaStage& mfma_stage(int wave);
int wave_of_cur();
}
template <typename AB, typename C>
inline C emu_mfma_32x32x8bf16(AB a, AB b, C c, int, int, int) {
    const int l = emu::lane_of_cur();
    emu::MfmaStage& st = emu::mfma_stage(emu::wave_of_cur());
    for (int t = 0; t < 4; ++t) {
        st.a[l][t] = (uint16_t)a[t];
        st.b[l][t] = (uint16_t)b[t];
    }
    emu::wave_op(emu::OP_BARRIER, 0, 0);
    const int j = l % 32, half = l / 32;
    C d = c;
    for (int r = 0; r < 16; ++r) {
        const int i = 8 * (r / 4) + 4 * half + r % 4;
        float acc = 0.0f;
        for (int k = 0; k < 8; ++k) {
            const int la = i + 32 * (k / 4), lb = j + 32 * (k / 4);
            const float x = __uint_as_float((uint32_t)st.a[la][k % 4] << 16);
            const float y = __uint_as_float((uint32_t)st.b[lb][k % 4] << 16);
            acc = __builtin_fmaf(x, y, acc);
        }
        d[r] = c[r] + acc;
    }
    emu::wave_op(emu::OP_BARRIER, 0, 0);
    return d;
}
#define __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(a, b, c, x, y, z) emu_mfma_32x32x8bf16(a, b, c, x, y, z)

inline float __uint_as_float(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t __float_as_uint(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float __int_as_float(int u) { float f; std::memcpy(&f, &u, 4); return f; }
inline int __float_as_int(float f) { int u; std::memcpy(&u, &f, 4); return u; }
inline long long __double_as_longlong(double d) { long long u; std::memcpy(&u, &d, 8); return u; }
inline double __longlong_as_double(long long u) { double d; std::memcpy(&d, &u, 8); return d; }
inline int __popcll(unsigned long long x) { return __builtin_popcountll(x); }
inline int __popc(unsigned x) { return __builtin_popcount(x); }
inline int __clzll(long long x) { return x ? __builtin_clzll((unsigned long long)x) : 64; }
inline int __ffsll(long long x) { return __builtin_ffsll(x); }
inline int __ffsll(unsigned long long x) { return __builtin_ffsll((long long)x); }

// Atomics live in emu.cpp, which has no basic-block hooks: a lane cannot be switched out
// between an atomic's read and its write.
#define EMU_ATOMICS(T)                  \
    T atomicAdd(T* p, T v);             \
    T atomicOr(T* p, T v);              \
    T atomicMax(T* p, T v);             \
    T atomicMin(T* p, T v);             \
    T atomicExch(T* p, T v);            \
    T atomicCAS(T* p, T c, T v);
EMU_ATOMICS(int)
EMU_ATOMICS(unsigned)
EMU_ATOMICS(unsigned long long)
EMU_ATOMICS(long long)
float atomicAdd(float* p, float v);
float atomicMax(float* p, float v);
float atomicExch(float* p, float v);

// host runtime stubs: synchronous, one device
inline hipError_t hipGetLastError() { hipError_t e = emu::g_last_error; emu::g_last_error = 0; return e; }
inline const char* hipGetErrorString(hipError_t) { return "emulated error"; }
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned) { *s = (hipStream_t)0x10; return hipSuccess; }
inline hipError_t hipStreamDestroy(hipStream_t) { return hipSuccess; }
inline hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) { *e = (hipEvent_t)0x20; return hipSuccess; }
inline hipError_t hipEventDestroy(hipEvent_t) { return hipSuccess; }
inline hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
inline hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t, unsigned) { return hipSuccess; }
inline hipError_t hipMemcpyAsync(void* d, const void* s, size_t n, hipMemcpyKind, hipStream_t) { std::memmove(d, s, n); return hipSuccess; }
#define HIP_SYMBOL(x) (x)
template <typename T>
inline hipError_t hipGetSymbolAddress(void** p, T& sym) { *p = (void*)&sym; return hipSuccess; }
