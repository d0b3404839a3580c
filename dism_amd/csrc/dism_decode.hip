// dism_decode.hip -- inference: query-reset starts for prefill, and the incremental decoder.
//
// Decoder.  The training readout splits every valid pair (key j <= query i, equal labels)
// into a length-1 part, sq_i^T M with M the running sum of sk_j (x) v_j over the label's keys,
// and corrections for bigram pairs (equal (previous, current) labels, L >= 2).  A decoder
// keeps exactly that state per (batch, head) row, so one new token costs O(R*DV) plus its
// bigram pairs -- no suffix automaton and no rebuilds:
//   * a label table (open addressing, `slots` entries): per label the running matrix M
//     [R][DV] fp32, the key count, the last key, and the list of its key positions in
//     ascending order (blocks of 64 positions from a per-row pool);
//   * the raw history: query/key labels and the sk, v rows (cache dtype);
//   * meta: position, pool blocks used, last query reset, error flag.
// A step processes the new tokens of every row in order: key first (M += sk (x) v, append to
// its label's list), then the query: y = sq^T M[label], the bigram partners among the keys of
// its label (key j >= 1 with k[j-1] == q[i-1]), their suffix walks (bounded by the last query
// reset), and the output -- the same fp32 sequence as the training forward
// (oracle/dism_cpu_model.c, orc_forward / orc_forward_reset), so a decoded token equals the
// forward's output at that position bit for bit.
//
// Mapping: one 64-lane wave per row (lane = value column for M and outputs, lane = candidate
// partner for the scans and walks).  Labels, counts and lists written by lane 0 are read by
// other lanes after an agent-scope fence per token.
#include "dism_path.h"

DISM_TU_LAYOUT(decode)

namespace dism {

constexpr int DEC_WAVES = 4;

__device__ __forceinline__ uint32_t label_hash(int32_t x) {
    uint32_t h = (uint32_t)x;
    h ^= h >> 16;
    h *= 0x7feb352du;
    h ^= h >> 15;
    h *= 0x846ca68bu;
    h ^= h >> 16;
    return h;
}

// Slot of label x in the row's table: the first slot on x's probe sequence that holds x or
// is empty (64 probes per round).  Returns the slot (or -1 if the table is full); found
// tells which.
__device__ __forceinline__ int probe(const int32_t* cnt, const int32_t* lab, int slots, int32_t x,
                                     bool& found) {
    const int lane = lane_id();
    const uint32_t mask = (uint32_t)slots - 1u, h0 = label_hash(x);
    for (int base = 0; base < slots; base += 64) {
        const int idx = (int)((h0 + (uint32_t)(base + lane)) & mask);
        const int c = cnt[idx];
        const bool hit = c > 0 && lab[idx] == x, empty = c == 0;
        const unsigned long long m = __ballot(hit || empty);
        if (m) {
            const int f = __ffsll((long long)m) - 1;
            found = __shfl((int)hit, f) != 0;
            return __shfl(idx, f);
        }
    }
    found = false;
    return -1;
}

__device__ __forceinline__ float wave_max_f(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}

template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * DEC_WAVES) void decode_kernel(DecodeArgs a) {
    constexpr int COLS = (DV + 63) / 64;
    const int lane = lane_id();
    const int bh = (int)blockIdx.x * DEC_WAVES + wave_id();
    if (bh >= a.rows) return;
    const int h = bh % a.H, b = bh / a.H;
    int32_t* meta = a.meta + (long)bh * 4;
    int pos = meta[0], pool_next = meta[1], last_reset = meta[2], err = meta[3];
    const long cap = a.cap;
    int32_t* qlab = a.qlab + bh * cap;
    int32_t* klab = a.klab + bh * cap;
    T* skh = reinterpret_cast<T*>(a.skh) + bh * cap * R;
    T* vh = reinterpret_cast<T*>(a.vh) + bh * cap * DV;
    int32_t* slot_label = a.slot_label + (long)bh * a.slots;
    int32_t* slot_cnt = a.slot_cnt + (long)bh * a.slots;
    int32_t* slot_last = a.slot_last + (long)bh * a.slots;
    float* Mrow = a.M + (long)bh * a.slots * (R * DV);
    int32_t* blocks = a.slot_blocks + (long)bh * a.slots * a.bcap;
    int32_t* pool = a.pool + (long)bh * a.pool_blocks * LIST_BLOCK;
    int32_t* scratch = a.scratch + bh * cap;
    const T* sk_in = reinterpret_cast<const T*>(a.sk);
    const T* v_in = reinterpret_cast<const T*>(a.v);
    const T* sq_in = reinterpret_cast<const T*>(a.sq);
    const float* tab = a.lut ? a.lut + (long)h * a.lut_stride : nullptr;

    for (int x = 0; x < a.n; ++x) {
        const int t = pos + x;
        const long lrow = (long)bh * a.n + x;                 // [B,H,n]
        const long irow = ((long)b * a.n + x) * a.H + h;      // [B,n,H,*]
        const int32_t lk = a.ik[lrow], lq = a.iq[lrow];
        if (a.reset && a.reset[lrow]) last_reset = t;
        // ---- history
        if (lane == 0) {
            qlab[t] = lq;
            klab[t] = lk;
        }
        for (int e = lane; e < R; e += 64) skh[(long)t * R + e] = sk_in[irow * R + e];
        for (int e = lane; e < DV; e += 64) vh[(long)t * DV + e] = v_in[irow * DV + e];
        // ---- key t: M[label] += sk (x) v, count, last, position list
        bool found;
        const int s = probe(slot_cnt, slot_label, a.slots, lk, found);
        if (s < 0) {
            err = 1;
        } else {
            float skr[R];
#pragma unroll
            for (int r = 0; r < R; ++r) skr[r] = load_elem<T>(sk_in, irow * R + r);
            float* Ms = Mrow + (long)s * (R * DV);
#pragma unroll
            for (int c = 0; c < COLS; ++c) {
                const int d = lane + 64 * c;
                if (d < DV) {
                    const float vd = load_elem<T>(v_in, irow * DV + d);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float m0 = found ? Ms[r * DV + d] : 0.0f;
                        Ms[r * DV + d] = __builtin_fmaf(skr[r], vd, m0);
                    }
                }
            }
            const int cnt0 = found ? slot_cnt[s] : 0;
            if (lane == 0) {
                int32_t* sb = blocks + (long)s * a.bcap;
                bool ok = true;
                if (cnt0 % LIST_BLOCK == 0) {
                    if (pool_next < a.pool_blocks) sb[cnt0 / LIST_BLOCK] = pool_next++;
                    else ok = false;
                }
                if (ok) {
                    pool[(long)sb[cnt0 / LIST_BLOCK] * LIST_BLOCK + cnt0 % LIST_BLOCK] = t;
                    slot_label[s] = lk;
                    slot_cnt[s] = cnt0 + 1;
                    slot_last[s] = t;
                } else {
                    err = 1;
                }
            }
            pool_next = __shfl(pool_next, 0);
            err = __shfl(err, 0);
        }
        __threadfence();  // lane 0's table, list and label writes before any lane reads them
        if (!a.out) continue;

        // ---- query t
        const int qs = probe(slot_cnt, slot_label, a.slots, lq, found);
        const bool have = qs >= 0 && found;
        const int cnt = have ? slot_cnt[qs] : 0;
        float sqr[R];
#pragma unroll
        for (int r = 0; r < R; ++r) sqr[r] = load_elem<T>(sq_in, irow * R + r);
        const float lut1 = tab[1];
        float m = (cnt > 0 && lut1 > 0.0f) ? lut1 : 0.0f;
        int np = 0;
        const int32_t* sb = have ? blocks + (long)qs * a.bcap : nullptr;
        const int lo = last_reset;
        // pass 1: candidates (keys of the query's label), bigram test, walks, row maximum
        if (have && t >= 1) {
            const int32_t pq = qlab[t - 1];
            for (int base = 0; base < cnt; base += 64) {
                const int xi = base + lane;
                int j = 0, L = 0;
                if (xi < cnt) {
                    j = pool[(long)sb[xi / LIST_BLOCK] * LIST_BLOCK + xi % LIST_BLOCK];
                    if (j >= 1 && klab[j - 1] == pq) {
                        int c = t - 1 >= lo ? 2 : 1;
                        while (t - c >= lo && j - c >= 0 && qlab[t - c] == klab[j - c]) ++c;
                        L = c;
                    }
                    scratch[xi] = L;
                }
                const unsigned long long pm = __ballot(L > 0);
                np += __popcll(pm);
                const float tl = L > 0 ? tab[L] : 0.0f;
                m = fmaxf(m, wave_max_f(tl));
            }
        }
        // pass 2: weights, corrections in ascending key order
        const float p1 = exp2_fp32(lut1 - m);
        float dp = 0.0f;
        float corr[COLS];
#pragma unroll
        for (int c = 0; c < COLS; ++c) corr[c] = 0.0f;
        if (np > 0) {
            for (int base = 0; base < cnt; base += 64) {
                const int xi = base + lane;
                int j = 0, L = 0;
                if (xi < cnt) {
                    L = scratch[xi];
                    j = pool[(long)sb[xi / LIST_BLOCK] * LIST_BLOCK + xi % LIST_BLOCK];
                }
                float p = 0.0f, cf = 0.0f;
                if (L > 0) {
                    p = exp2_fp32(tab[L] - m);
                    float sdot = 0.0f;
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        sdot = __builtin_fmaf(sqr[r], load_elem<T>(skh, (long)j * R + r), sdot);
                    cf = (p - p1) * sdot;
                }
                unsigned long long pm = __ballot(L > 0);
                while (pm) {
                    const int e = __ffsll((long long)pm) - 1;
                    pm &= pm - 1;
                    dp = dp + readlane_f(p, e);
                    const float ce = readlane_f(cf, e);
                    const int je = readlane_i(j, e);
#pragma unroll
                    for (int c = 0; c < COLS; ++c) {
                        const int d = lane + 64 * c;
                        if (d < DV)
                            corr[c] = __builtin_fmaf(ce, load_elem<T>(vh, (long)je * DV + d),
                                                     corr[c]);
                    }
                }
            }
        }
        // ---- output
        const float den = (exp2_fp32(-m) + (float)(cnt - np) * p1) + dp;
        const float rden = 1.0f / den;
        const float* Ms = have ? Mrow + (long)qs * (R * DV) : nullptr;
#pragma unroll
        for (int c = 0; c < COLS; ++c) {
            const int d = lane + 64 * c;
            if (d >= DV) continue;
            float y = 0.0f;
            if (have) {
#pragma unroll
                for (int r = 0; r < R; ++r) y = __builtin_fmaf(sqr[r], Ms[r * DV + d], y);
            }
            a.out[irow * DV + d] = __builtin_fmaf(p1, y, corr[c]) * rden;
        }
        if (a.lse2 && lane == 0) a.lse2[lrow] = m + log2_fp32(den);
    }
    if (lane == 0) {
        meta[0] = pos + a.n;
        meta[1] = pool_next;
        meta[2] = last_reset;
        meta[3] = err;
    }
}

// ---------------------------------------------------------------------------------------
// Parallel prime: the decoder state of a whole prompt (keys only) from the prompt's combined
// label order (dism_hard_prepare on the prompt, padded past n; entries at positions >= n are
// skipped).  One wave per (row, top-digit bucket) as in the label scans; for every label
// group with keys it claims a table slot (atomic CAS of the slot's key count, so groups of
// one row never collide), takes list blocks from the row's pool (atomic add), writes the key
// positions in ascending order and folds M over the keys in position order -- the fp32
// chain of the serial key steps, so the state decodes exactly like a serially primed one.
// History rows, labels and the last reset are written per position.
template <typename T, int R, int DV>
__global__ __launch_bounds__(64 * DEC_WAVES) void prime_kernel(DecodeArgs a, Orders o,
                                                               int npad) {
    constexpr int COLS = (DV + 63) / 64;
    const int lane = lane_id();
    const long item = (long)blockIdx.x * DEC_WAVES + wave_id();
    const int bh = (int)(item >> 8), bucket = (int)(item & 255);
    if (bh >= a.rows) return;
    const int h = bh % a.H, b = bh / a.H;
    const long so = (long)bh * npad, cap = a.cap;
    const int32_t* corder = o.corder + 2 * so;
    const int32_t* clab = o.clab + 2 * so;
    const int c0 = o.ctab[(long)bh * 257 + bucket], c1 = o.ctab[(long)bh * 257 + bucket + 1];
    int32_t* meta = a.meta + (long)bh * 4;
    int32_t* qlab = a.qlab + bh * cap;
    int32_t* klab = a.klab + bh * cap;
    T* skh = reinterpret_cast<T*>(a.skh) + bh * cap * R;
    T* vh = reinterpret_cast<T*>(a.vh) + bh * cap * DV;
    int32_t* slot_label = a.slot_label + (long)bh * a.slots;
    int32_t* slot_cnt = a.slot_cnt + (long)bh * a.slots;
    int32_t* slot_last = a.slot_last + (long)bh * a.slots;
    float* Mrow = a.M + (long)bh * a.slots * (R * DV);
    int32_t* blocks = a.slot_blocks + (long)bh * a.slots * a.bcap;
    int32_t* pool = a.pool + (long)bh * a.pool_blocks * LIST_BLOCK;
    const T* sk_in = reinterpret_cast<const T*>(a.sk);
    const T* v_in = reinterpret_cast<const T*>(a.v);
    const unsigned long long below = lane ? (~0ull >> (64 - lane)) : 0ull;
    // history and resets, lane-parallel over the bucket's entries
    for (int x = c0 + lane; x < c1; x += 64) {
        const int e = corder[x], p = e >> 1;
        if (p >= a.n) continue;
        const long lrow = (long)bh * a.n + p, irow = ((long)b * a.n + p) * a.H + h;
        if (e & 1) {
            qlab[p] = a.iq[lrow];
            if (a.reset && a.reset[lrow]) atomicMax(meta + 2, p);
        } else {
            klab[p] = a.ik[lrow];
            for (int r = 0; r < R; ++r) skh[(long)p * R + r] = sk_in[irow * R + r];
            for (int d = 0; d < DV; ++d) vh[(long)p * DV + d] = v_in[irow * DV + d];
        }
    }
    int rs = __builtin_amdgcn_readfirstlane(c0);
    const int ce = __builtin_amdgcn_readfirstlane(c1);
    while (rs < ce) {
        const uint32_t lbl = (uint32_t)__builtin_amdgcn_readfirstlane(clab[rs]);
        const int re = __builtin_amdgcn_readfirstlane(
            (uint32_t)clab[ce - 1] == lbl ? ce : upper_label(clab, rs + 1, ce, lbl));
        // keys of the group (entries 2p, p < n), in position order
        int nk = 0;
        for (int x0 = rs; x0 < re; x0 += 64) {
            const int x = x0 + lane;
            const int e = x < re ? corder[x] : 1;
            nk += __popcll(__ballot(!(e & 1) && (e >> 1) < a.n));
        }
        if (nk > 0) {
            const int32_t label = (int32_t)lbl;
            int s = -1;
            if (lane == 0) {  // claim the first free slot on the label's probe sequence
                const uint32_t mask = (uint32_t)a.slots - 1u, h0 = label_hash(label);
                for (int t = 0; t < a.slots; ++t) {
                    const int idx = (int)((h0 + (uint32_t)t) & mask);
                    if (atomicCAS(slot_cnt + idx, 0, nk) == 0) {
                        s = idx;
                        break;
                    }
                }
                if (s < 0) atomicExch(meta + 3, 1);
            }
            s = __shfl(s, 0);
            if (s >= 0) {
                const int nb = (nk + LIST_BLOCK - 1) / LIST_BLOCK;
                int base = 0;
                if (lane == 0) base = atomicAdd(meta + 1, nb);
                base = __shfl(base, 0);
                int32_t* sb = blocks + (long)s * a.bcap;
                for (int t = lane; t < nb; t += 64) sb[t] = base + t;
                float M[R][COLS];
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int c = 0; c < COLS; ++c) M[r][c] = 0.0f;
                int kseen = 0, last = 0;
                for (int x0 = rs; x0 < re; x0 += 64) {
                    const int x = x0 + lane;
                    const int e = x < re ? corder[x] : 1;
                    const bool isk = !(e & 1) && (e >> 1) < a.n;
                    const unsigned long long km = __ballot(isk);
                    if (isk) {
                        const int xi = kseen + __popcll(km & below);
                        pool[(long)(base + xi / LIST_BLOCK) * LIST_BLOCK + xi % LIST_BLOCK] =
                            e >> 1;
                    }
                    // M over this window's keys, in order
                    unsigned long long mm = km;
                    while (mm) {
                        const int l = __ffsll((long long)mm) - 1;
                        mm &= mm - 1;
                        const int p = readlane_i(e, l) >> 1;
                        const long irow = ((long)b * a.n + p) * a.H + h;
                        float skr[R];
#pragma unroll
                        for (int r = 0; r < R; ++r) skr[r] = load_elem<T>(sk_in, irow * R + r);
#pragma unroll
                        for (int c = 0; c < COLS; ++c) {
                            const int d = lane + 64 * c;
                            const float vd = d < DV ? load_elem<T>(v_in, irow * DV + d) : 0.0f;
#pragma unroll
                            for (int r = 0; r < R; ++r)
                                M[r][c] = __builtin_fmaf(skr[r], vd, M[r][c]);
                        }
                        last = p;
                    }
                    kseen += __popcll(km);
                }
                float* Ms = Mrow + (long)s * (R * DV);
#pragma unroll
                for (int c = 0; c < COLS; ++c) {
                    const int d = lane + 64 * c;
                    if (d < DV) {
#pragma unroll
                        for (int r = 0; r < R; ++r) Ms[r * DV + d] = M[r][c];
                    }
                }
                if (lane == 0) {
                    slot_label[s] = label;
                    slot_last[s] = last;
                }
            }
        }
        rs = re;
    }
    if (item == (long)bh * 256 && lane == 0) meta[0] = a.n;  // one writer per row
}

template <typename T, int R>
static hipError_t decode_dv(const DecodeArgs& a, hipStream_t s) {
    const unsigned grid = (unsigned)((a.rows + DEC_WAVES - 1) / DEC_WAVES);
    const dim3 block(64 * DEC_WAVES);
    switch (a.DV) {
        case 32: hipLaunchKernelGGL((decode_kernel<T, R, 32>), dim3(grid), block, 0, s, a); break;
        case 64: hipLaunchKernelGGL((decode_kernel<T, R, 64>), dim3(grid), block, 0, s, a); break;
        case 128: hipLaunchKernelGGL((decode_kernel<T, R, 128>), dim3(grid), block, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename T>
static hipError_t decode_r(const DecodeArgs& a, hipStream_t s) {
    switch (a.R) {
        case 2: return decode_dv<T, 2>(a, s);
        case 4: return decode_dv<T, 4>(a, s);
        case 8: return decode_dv<T, 8>(a, s);
        case 16: return decode_dv<T, 16>(a, s);
        case 32: return decode_dv<T, 32>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <typename T, int R>
static hipError_t prime_dv(const DecodeArgs& a, const Orders& o, int npad, hipStream_t s) {
    const unsigned grid = (unsigned)((256L * a.rows + DEC_WAVES - 1) / DEC_WAVES);
    const dim3 block(64 * DEC_WAVES);
    switch (a.DV) {
        case 32:
            hipLaunchKernelGGL((prime_kernel<T, R, 32>), dim3(grid), block, 0, s, a, o, npad);
            break;
        case 64:
            hipLaunchKernelGGL((prime_kernel<T, R, 64>), dim3(grid), block, 0, s, a, o, npad);
            break;
        case 128:
            hipLaunchKernelGGL((prime_kernel<T, R, 128>), dim3(grid), block, 0, s, a, o, npad);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <typename T>
static hipError_t prime_r(const DecodeArgs& a, const Orders& o, int npad, hipStream_t s) {
    switch (a.R) {
        case 2: return prime_dv<T, 2>(a, o, npad, s);
        case 4: return prime_dv<T, 4>(a, o, npad, s);
        case 8: return prime_dv<T, 8>(a, o, npad, s);
        case 16: return prime_dv<T, 16>(a, o, npad, s);
        case 32: return prime_dv<T, 32>(a, o, npad, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_prime(const DecodeArgs& a, const Orders& o, int npad, int dtype,
                        hipStream_t s) {
    if (dtype == DTYPE_BF16) return prime_r<bf16_t>(a, o, npad, s);
    if (dtype == DTYPE_F32) return prime_r<float>(a, o, npad, s);
    return hipErrorInvalidValue;
}

hipError_t launch_decode(const DecodeArgs& a, int dtype, hipStream_t s) {
    if (dtype == DTYPE_BF16) return decode_r<bf16_t>(a, s);
    if (dtype == DTYPE_F32) return decode_r<float>(a, s);
    return hipErrorInvalidValue;
}

// rows of n labels -> rows of npad labels (0 past n)
__global__ __launch_bounds__(256) void pad_labels_kernel(const int32_t* __restrict__ src,
                                                         long rows, long n, long npad,
                                                         int32_t* __restrict__ dst) {
    const long x = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (x >= rows * npad) return;
    const long r = x / npad, p = x - r * npad;
    dst[x] = p < n ? src[r * n + p] : 0;
}

hipError_t launch_pad_labels(const int32_t* src, long rows, long n, long npad, int32_t* dst,
                             hipStream_t s) {
    hipLaunchKernelGGL(pad_labels_kernel, dim3((unsigned)((rows * npad + 255) / 256)), dim3(256),
                       0, s, src, rows, n, npad, dst);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Query-reset starts for prefill: wlo[bh, i] = the last position r <= i with reset[bh, r],
// else 0.  One block per row, chunked block max-scan.
constexpr int RS_THREADS = 1024, RS_ITEMS = 4;

__global__ __launch_bounds__(RS_THREADS) void reset_starts_kernel(
    const uint8_t* __restrict__ reset, long n, int32_t* __restrict__ wlo) {
    __shared__ int s_wave[RS_THREADS / 64];
    __shared__ int s_carry;
    const long row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint8_t* rs = reset + row * n;
    int32_t* out = wlo + row * n;
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (long base = 0; base < n; base += (long)RS_THREADS * RS_ITEMS) {
        const long x0 = base + (long)tid * RS_ITEMS;
        int v[RS_ITEMS], run = 0;
#pragma unroll
        for (int u = 0; u < RS_ITEMS; ++u) {
            const long x = x0 + u;
            if (x < n && rs[x]) run = (int)x;
            v[u] = run;
        }
        int incl = run;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl = y > incl ? y : incl;
        }
        if (lane == 63) s_wave[wave] = incl;
        __syncthreads();
        int before = s_carry;
        for (int w = 0; w < wave; ++w) before = s_wave[w] > before ? s_wave[w] : before;
        int excl = __shfl_up(incl, 1);
        if (lane == 0) excl = 0;
        const int prefix = excl > before ? excl : before;
#pragma unroll
        for (int u = 0; u < RS_ITEMS; ++u) {
            const long x = x0 + u;
            if (x < n) out[x] = v[u] > prefix ? v[u] : prefix;
        }
        __syncthreads();
        if (tid == RS_THREADS - 1) s_carry = prefix > incl ? prefix : incl;
        __syncthreads();
    }
}

hipError_t launch_reset_starts(const uint8_t* reset, long rows, long n, int32_t* wlo,
                               hipStream_t s) {
    hipLaunchKernelGGL(reset_starts_kernel, dim3((unsigned)rows), dim3(RS_THREADS), 0, s, reset,
                       n, wlo);
    return hipGetLastError();
}

}  // namespace dism
