// dism_sweep.h -- the symbol-bitmask sweep shared by the forward and backward kernels.
//
// A workgroup of 256 lanes owns 256 consecutive "owner" positions of one (batch, head) row:
// query rows for the forward / dSQ sweep, keys for the dV / dSK sweep.  The opposite side
// ("partners": keys, resp. queries) is streamed through LDS in tiles of KT positions.  For
// each tile the workgroup builds a 256-symbol bitmask table in LDS:
//     table[s][w] bit b  <=>  label(partner k0 + 32w + b) & 255 == s
// so one ds_read_b128 of table[label(owner) & 255] yields the prefiltered match mask of an
// owner against 128 partners.  Each candidate bit is verified against the full int32
// partner label (also staged in LDS) and handed to the caller's per-match functor in
// ascending partner order.  For random labels over an alphabet of A symbols only ~1/A of
// the pairs reach the functor; the integer scan itself costs ~3 VALU ops per 128 pairs.
#pragma once
#include "dism_device.h"

namespace dism {

constexpr int OWNERS = 256;               // lanes per workgroup
constexpr int KT = 1024;                  // partners per LDS tile
constexpr int TSTR = KT / 32 + 4;         // words per symbol row (+4: bank spread, 16B aligned)

struct SweepShared {
    uint32_t table[SYMBOLS * TSTR];
    int32_t labels[KT];
};

// Build the bitmask table for partners [p0, p0 + KT) clipped to [lo, hi].
__device__ __forceinline__ void build_table(SweepShared& sh, const int32_t* __restrict__ lab,
                                            int p0, int lo, int hi) {
    __syncthreads();
    uint4* t4 = reinterpret_cast<uint4*>(sh.table);
    for (int x = threadIdx.x; x < SYMBOLS * TSTR / 4; x += OWNERS) t4[x] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    for (int u = threadIdx.x; u < KT; u += OWNERS) {
        int p = p0 + u;
        if (p >= lo && p <= hi) {
            int l = lab[p];
            sh.labels[u] = l;
            atomicOr(&sh.table[(l & (SYMBOLS - 1)) * TSTR + (u >> 5)], 1u << (u & 31));
        }
    }
    __syncthreads();
}

// Visit the verified matches of one owner inside the current tile, ascending partner order.
// Partners u in [ulo, uhi) (tile-local indices) are eligible.
template <typename F>
__device__ __forceinline__ void visit_tile(const SweepShared& sh, int label, int ulo, int uhi,
                                           F&& on_match) {
    if (uhi > KT) uhi = KT;
    if (ulo < 0) ulo = 0;
    if (ulo >= uhi) return;
    const uint32_t* row = sh.table + (label & (SYMBOLS - 1)) * TSTR;
    int wbeg = (ulo >> 5) & ~3;
    int wend = (uhi + 31) >> 5;
    for (int w = wbeg; w < wend; w += 4) {
        uint4 mm = *reinterpret_cast<const uint4*>(row + w);
        uint32_t c[4] = {mm.x, mm.y, mm.z, mm.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int base = 32 * (w + t);
            int hiv = uhi - base;  // eligible bits below hiv
            int lov = ulo - base;  // eligible bits at or above lov
            uint32_t m = c[t];
            m = hiv <= 0 ? 0u : (hiv >= 32 ? m : m & ((1u << hiv) - 1u));
            m = lov >= 32 ? 0u : (lov <= 0 ? m : m & ~((1u << lov) - 1u));
            c[t] = m;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            while (c[t]) {
                int bit = __builtin_ctz(c[t]);
                c[t] &= c[t] - 1u;
                int u = 32 * (w + t) + bit;
                if (sh.labels[u] == label) on_match(u);
            }
        }
    }
}

}  // namespace dism
