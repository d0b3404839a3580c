// dism_sweep.h -- work decomposition shared by the bucketed sweep kernels.
//
// Positions of each (batch, head) row are grouped by symbol (dism_bucket.hip).  A wave owns
// one chunk of up to 64 "owner" positions of one bucket -- query rows for the forward and
// the dSQ sweep, keys for the dV/dSK sweep -- one owner per lane, and walks the opposite
// side's bucket of the same symbol ("partners") in ascending position order with a
// wave-uniform loop.  Partner data (labels, readout/value rows) is therefore wave-uniform and
// read through the scalar path; only the per-owner arithmetic is per lane.  A pair is a match
// when the full int32 labels agree and it is causal (key <= query); other pairs of the loop
// contribute exact zeros.
#pragma once
#include <type_traits>

#include "dism_device.h"
#include "dism_launch.h"

namespace dism {

struct Chunk {
    int bh, b, h;
    int sym;
    int first;    // index of the chunk's first owner in the owner side's position list
    int count;    // owners in this chunk (1..64)
    int pbeg;     // partner bucket [pbeg, pend) in the partner side's position list
    int pend;
};

// Work-item index of this workgroup with an XCD-contiguous mapping: workgroups are dispatched
// round-robin over the 8 XCDs, so consecutive work items (same (b,h) row, whose partner data
// then stays in one XCD's L2) are given to workgroups of one XCD.  grid is a multiple of 8.
__device__ __forceinline__ int xcd_work_item() {
    const int g = (int)gridDim.x, x = (int)blockIdx.x;
    return (x & 7) * (g >> 3) + (x >> 3);
}

// Locate the chunk of work item w; false for padding items.  key_owner selects the side.
__device__ __forceinline__ bool locate_chunk(const SweepCommon& c, int w, bool key_owner,
                                             Chunk& ch) {
    const int bh = w / c.slots;
    if (bh >= c.B * c.H) return false;
    const int slot = w - bh * c.slots;
    const int32_t* cs = (key_owner ? c.kcs : c.qcs) + (long)bh * (BUCKETS + 1);
    if (slot >= cs[BUCKETS]) return false;
    int lo = 0, hi = BUCKETS;  // cs[lo] <= slot < cs[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cs[mid] <= slot) lo = mid; else hi = mid;
    }
    const int32_t* oo = (key_owner ? c.koff : c.qoff) + (long)bh * (BUCKETS + 1);
    const int32_t* po = (key_owner ? c.qoff : c.koff) + (long)bh * (BUCKETS + 1);
    ch.bh = bh;
    ch.b = bh / c.H;
    ch.h = bh - ch.b * c.H;
    ch.sym = lo;
    ch.first = oo[lo] + (slot - cs[lo]) * CHUNK;
    const int left = oo[lo + 1] - ch.first;
    ch.count = left < CHUNK ? left : CHUNK;
    ch.pbeg = po[lo];
    ch.pend = po[lo + 1];
    return true;
}

// Scalar-path view of read-only global memory: loads through the constant address space with
// a wave-uniform address become s_load instructions and land in SGPRs, where VALU
// instructions can read them directly as operands.
template <typename T>
using cptr = const __attribute__((address_space(4))) T*;

template <typename T>
__device__ __forceinline__ cptr<T> as_const(const T* p) {
    return (cptr<T>)(p);
}

// N raw 32-bit words of a wave-uniform row.
template <int N>
struct SRow {
    uint32_t w[N];
};

template <int N>
__device__ __forceinline__ SRow<N> srow_load(cptr<uint32_t> q) {
    SRow<N> r;
#pragma unroll
    for (int c = 0; c < N; ++c) r.w[c] = q[c];
    return r;
}

// Element e (fp32) of a row of T stored as raw words.
template <typename T, int N>
__device__ __forceinline__ float srow_get(const SRow<N>& r, int e) {
    if constexpr (sizeof(T) == 2) {
        const uint32_t x = r.w[e >> 1];
        return __uint_as_float((e & 1) ? (x & 0xFFFF0000u) : (x << 16));
    } else {
        return __uint_as_float(r.w[e]);
    }
}

// words needed for n elements of T
template <typename T>
constexpr int words(int n) {
    return sizeof(T) == 2 ? (n + 1) / 2 : n;
}

// Value dimensions per wave: the largest block of DV whose partner row (readout + value words)
// fits a 24-word scalar budget, so the current and the prefetched partner both stay in SGPRs.
template <typename T, int R, int DV>
constexpr int value_block() {
    int b = DV < 64 ? DV : 64;
    while (b > 8 && (words<T>(R) + words<T>(b) > 24 || DV % b != 0)) b /= 2;
    return b;
}

}  // namespace dism
