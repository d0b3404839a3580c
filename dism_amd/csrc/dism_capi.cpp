// dism_capi.cpp -- extern "C" boundary of libdism_hip.so: argument validation, workspace
// layout, launch dispatch, thread-local error text.  Declarations and reference mapping:
// include/dism_hard.h.
#include <hip/hip_runtime.h>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

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

// Layout fingerprints of the translation units (DISM_TU_LAYOUT, dism_launch.h): every kernel
// unit must have been compiled against this unit's argument-struct layout.
#define DISM_TU_LIST(X)                                                                    \
    X(aux) X(sort) X(msort) X(pairs) X(scan) X(packed) X(dense) X(levels) X(prefix)          \
    X(prefix_rows) X(prefix_keys) X(decode) X(vocab)
#define DISM_TU_DECL(tu) extern "C" const unsigned long long dism_layout_##tu;
DISM_TU_LIST(DISM_TU_DECL)
#undef DISM_TU_DECL

std::string layout_mismatch() {
    std::string bad;
    constexpr unsigned long long want = dism::layout_fingerprint();
#define DISM_TU_CMP(tu)                                                                     \
    if (dism_layout_##tu != want) bad += (bad.empty() ? "" : ", ") + std::string("dism_" #tu);
    DISM_TU_LIST(DISM_TU_CMP)
#undef DISM_TU_CMP
    return bad;
}

// DISM_OK once every unit matches (checked once per process), else an error naming the units
int32_t layout_guard() {
    static const std::string bad = layout_mismatch();
    if (bad.empty()) return DISM_OK;
    return fail(DISM_ERR_INVALID,
                "library linked from objects with mismatched argument-struct layouts (stale: "
                "%s); rebuild every translation unit", bad.c_str());
}

bool dims_ok(int64_t B, int64_t N, int64_t H) {
    return B > 0 && H > 0 && N > 0 && N <= INT_MAX / 64 && B * H <= 65535;
}
bool rdv_ok(int32_t R, int32_t DV) {
    return (R == 2 || R == 4 || R == 8 || R == 16 || R == 32) &&
           (DV == 32 || DV == 64 || DV == 128);
}
bool dtype_ok(int32_t d) { return d == DISM_BF16 || d == DISM_F32; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Workspace layout (each section 256-byte aligned).
//   orders: label order and bigram order of both sides (dism_sort.hip) + sort scratch
//   pnb/prow: per query row bigram-pair count and record (layout: dism_launch.h)
struct Layout {
    int64_t corder, clab, ctab, bpos[2], blab[2], bplab[2], btab[2], shift, tmp[3];
    int64_t stage[2][2], bhcount[2], own[2], ocount, mode, onebyte;
    int64_t pnb, prow, mcount, mdig, dflag, dlist, dcount, dbound, dcost, runs, runcnt;
    int64_t lvent, lvlc, lvlf, lvlk, lvmeta, lvq, lvqidx, lvkidx, lvF, lvFk, lvP, lvQ, lvY, lvZ, lvK;  // -1: none
    int64_t pxT, pxB, pxU, pxS, pxR, pxK, pxKR, pxE, pxL;  // -1: none
    int64_t total;
    int prow_stride;
};

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Side streams (default priority, non-blocking) with their fork/join events, one set per
// concurrent call: a per-device pool that a call borrows from and returns to, so the number of
// streams and events is bounded by the largest number of simultaneous calls on a device,
// however many threads call over the process's lifetime.  The pool lives until the process
// ends.  A call without a set (HIP could not create one) runs its launches serially.
struct SideStream {
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    hipEvent_t mid = nullptr;  // a point inside the side chain the caller's stream waits for
};

constexpr int MAX_DEVICES = 64;
std::mutex g_side_mutex;
std::vector<SideStream*> g_side_free[MAX_DEVICES];

class SideLease {
  public:
    SideLease() {
        if (hipGetDevice(&dev_) != hipSuccess || dev_ < 0 || dev_ >= MAX_DEVICES) return;
        {
            std::lock_guard<std::mutex> lock(g_side_mutex);
            if (!g_side_free[dev_].empty()) {
                s_ = g_side_free[dev_].back();
                g_side_free[dev_].pop_back();
                return;
            }
        }
        SideStream* c = new SideStream;
        if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
            delete c;
            return;
        }
        if (hipEventCreateWithFlags(&c->fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&c->join, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&c->mid, hipEventDisableTiming) != hipSuccess) {
            if (c->fork) hipEventDestroy(c->fork);
            if (c->join) hipEventDestroy(c->join);
            hipStreamDestroy(c->stream);
            delete c;
            return;
        }
        s_ = c;
    }
    ~SideLease() {
        if (!s_) return;
        std::lock_guard<std::mutex> lock(g_side_mutex);
        g_side_free[dev_].push_back(s_);
    }
    SideLease(const SideLease&) = delete;
    SideLease& operator=(const SideLease&) = delete;
    SideStream* get() const { return s_; }

  private:
    int dev_ = -1;
    SideStream* s_ = nullptr;
};

// A leased side stream forked from `s` for the backward's pairless-mode kernels (dense
// tiles, level rows, prefix rows): their rows are disjoint from the label scans' rows, so
// they run beside the scan instead of ahead of it on the same chain (at the headline shape
// they find no rows, but each launch still waits for free compute units).  join() records
// the side stream's work and makes `s` wait for it; without a side stream everything stays
// on `s`.
class PairlessFork {
  public:
    explicit PairlessFork(hipStream_t s) : s_(s) {
        side_ = lease_.get();
        if (side_ && (hipEventRecord(side_->fork, s_) != hipSuccess ||
                      hipStreamWaitEvent(side_->stream, side_->fork, 0) != hipSuccess))
            side_ = nullptr;
    }
    hipStream_t side() const { return side_ ? side_->stream : s_; }
    bool join() {
        if (!side_) return true;
        const bool ok = hipEventRecord(side_->join, side_->stream) == hipSuccess &&
                        hipStreamWaitEvent(s_, side_->join, 0) == hipSuccess;
        side_ = nullptr;
        return ok;
    }
    ~PairlessFork() { join(); }
    PairlessFork(const PairlessFork&) = delete;
    PairlessFork& operator=(const PairlessFork&) = delete;

  private:
    hipStream_t s_;
    SideLease lease_;
    SideStream* side_ = nullptr;
};

Layout layout(int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV) {
    Layout L;
    const int64_t BH = B * H;
    L.prow_stride = (DV + dism::PREC_Y > R + 4 ? DV + dism::PREC_Y : R + 4);
    int64_t o = 0;
    auto take = [&](int64_t bytes) {
        int64_t a = o;
        o += align256(bytes);
        return a;
    };
    L.corder = take(BH * 2 * N * 4);
    L.clab = take(BH * 2 * N * 4);
    L.ctab = take(BH * 257 * 4);
    for (int s = 0; s < 2; ++s) {
        L.bpos[s] = take(BH * N * 4);
        L.blab[s] = take(BH * N * 4);
        L.bplab[s] = take(BH * N * 4);
        L.btab[s] = take(BH * 257 * 4);
    }
    L.shift = take(BH * 4);
    for (int s = 0; s < 2; ++s) {
        L.stage[s][0] = take(BH * N * 16);
        L.stage[s][1] = take(BH * N * 16);
        L.bhcount[s] = take(BH * 16);
        L.own[s] = take(BH * N * 16);
    }
    L.ocount = take(8 * 4);
    L.mode = take(BH * 4);
    L.onebyte = take(BH * 4);
    L.mcount = take(3 * BH * 256 * dism::MSORT_SEGMENTS * 4);
    L.mdig = take(BH * (32 + 8) * 4);
    L.tmp[0] = take(BH * 2 * N * 4);
    L.tmp[1] = take(BH * N * 4);
    L.tmp[2] = take(BH * N * 4);
    L.pnb = take(BH * N * 4);
    L.prow = take(BH * N * L.prow_stride * 4);
    L.dflag = take(BH * 4);
    L.dlist = take(4 * BH * 4);
    L.dcount = take(4 * 4);
    L.dbound = take(N <= dism::DENSE_MAX_N ? BH * dism::dense_row_entries((int)N) * 2 : 0);
    L.dcost = take(BH * 8);
    L.runs = take(BH * dism::RUN_CAP * 16);
    L.runcnt = take(BH * 4);
    // level rows (dism_levels.hip) only where they can occur
    const bool lv = N <= dism::LEVEL_MAX_N && (int64_t)R * DV <= dism::LEVEL_RDV;
    const int64_t lent = (int64_t)dism::LEVEL_BUDGET * N, lmat = dism::LEVEL_MAX * N;
    const int64_t lseg = dism::level_segs(N) * R * DV * 4;
    L.lvent = lv ? take(BH * lmat * 2 * 4) : -1;
    L.lvlc = lv ? take(BH * (dism::LEVEL_MAX + 2) * 4) : -1;
    L.lvlf = lv ? take(BH * (dism::LEVEL_MAX + 1) * N) : -1;
    L.lvlk = lv ? take(BH * lmat * 2) : -1;
    L.lvmeta = lv ? take(BH * dism::LEVEL_META * 4) : -1;
    L.lvqidx = lv ? take(BH * lmat * 2) : -1;
    L.lvkidx = lv ? take(BH * lmat * 2) : -1;
    L.lvF = lv ? take(BH * dism::level_segs(N)) : -1;
    L.lvFk = lv ? take(BH * dism::level_segs(N)) : -1;
    L.lvq = lv ? take(BH * N * 16) : -1;
    L.lvP = lv ? take(BH * lseg) : -1;
    L.lvQ = lv ? take(BH * lseg) : -1;
    L.lvY = lv ? take(BH * lent * DV * 4) : -1;
    L.lvZ = lv ? take(BH * lent * R * 4) : -1;
    L.lvK = lv ? take(BH * lent * R * 4) : -1;
    // prefix rows (dism_prefix.hip) wherever dense rows can occur
    const bool px = N <= dism::DENSE_MAX_N;
    const int64_t pseg = px ? (int64_t)dism::px_segs((int)N) : 0;
    L.pxT = px ? take(BH * pseg * R * DV * 4) : -1;
    L.pxB = px ? take(BH * pseg * R * DV * 4) : -1;
    L.pxU = px ? take(BH * pseg * R * DV * 4) : -1;
    L.pxS = px ? take(BH * pseg * 16) : -1;
    L.pxR = px ? take(BH * pseg * 16) : -1;
    L.pxK = px ? take(BH * pseg * 8) : -1;
    L.pxKR = px ? take(BH * pseg * 8) : -1;
    L.pxE = px ? take(BH * 2 * N * 4) : -1;
    L.pxL = px ? take(BH * 2 * N * 4) : -1;
    L.total = o;
    return L;
}

template <typename P>
P* at(void* ws, int64_t off) {
    return reinterpret_cast<P*>(reinterpret_cast<char*>(ws) + off);
}

dism::Orders orders(const Layout& L, void* ws) {
    dism::Orders o;
    o.corder = at<int32_t>(ws, L.corder);
    o.clab = at<int32_t>(ws, L.clab);
    o.ctab = at<int32_t>(ws, L.ctab);
    for (int s = 0; s < 2; ++s) {
        o.bpos[s] = at<int32_t>(ws, L.bpos[s]);
        o.blab[s] = at<int32_t>(ws, L.blab[s]);
        o.bplab[s] = at<int32_t>(ws, L.bplab[s]);
        o.btab[s] = at<int32_t>(ws, L.btab[s]);
    }
    o.shift = at<int32_t>(ws, L.shift);
    for (int s = 0; s < 2; ++s) {
        o.stage[s][0] = at<int4>(ws, L.stage[s][0]);
        o.stage[s][1] = at<int4>(ws, L.stage[s][1]);
        o.bhcount[s] = at<int32_t>(ws, L.bhcount[s]);
        o.own[s] = at<int4>(ws, L.own[s]);
    }
    o.ocount = at<int32_t>(ws, L.ocount);
    o.mode = at<int32_t>(ws, L.mode);
    o.onebyte = at<int32_t>(ws, L.onebyte);
    o.mcount = at<int32_t>(ws, L.mcount);
    o.mdig = at<int32_t>(ws, L.mdig);
    o.dflag = at<int32_t>(ws, L.dflag);
    o.dlist = at<int32_t>(ws, L.dlist);
    o.dcount = at<int32_t>(ws, L.dcount);
    o.dbound = at<uint16_t>(ws, L.dbound);
    o.dcost = at<unsigned long long>(ws, L.dcost);
    o.runs = at<int4>(ws, L.runs);
    o.runcnt = at<int32_t>(ws, L.runcnt);
    auto opt = [&](int64_t off) { return off < 0 ? nullptr : at<char>(ws, off); };
    o.lvent = reinterpret_cast<int32_t*>(opt(L.lvent));
    o.lvlc = reinterpret_cast<int32_t*>(opt(L.lvlc));
    o.lvlf = reinterpret_cast<uint8_t*>(opt(L.lvlf));
    o.lvlk = reinterpret_cast<uint16_t*>(opt(L.lvlk));
    o.lvmeta = reinterpret_cast<int32_t*>(opt(L.lvmeta));
    o.lvqidx = reinterpret_cast<uint16_t*>(opt(L.lvqidx));
    o.lvkidx = reinterpret_cast<uint16_t*>(opt(L.lvkidx));
    o.lvF = reinterpret_cast<uint8_t*>(opt(L.lvF));
    o.lvFk = reinterpret_cast<uint8_t*>(opt(L.lvFk));
    o.lvq = reinterpret_cast<int4*>(opt(L.lvq));
    o.lvP = reinterpret_cast<float*>(opt(L.lvP));
    o.lvQ = reinterpret_cast<float*>(opt(L.lvQ));
    o.lvY = reinterpret_cast<float*>(opt(L.lvY));
    o.lvZ = reinterpret_cast<float*>(opt(L.lvZ));
    o.lvK = reinterpret_cast<float*>(opt(L.lvK));
    o.pxT = reinterpret_cast<float*>(opt(L.pxT));
    o.pxB = reinterpret_cast<float*>(opt(L.pxB));
    o.pxU = reinterpret_cast<float*>(opt(L.pxU));
    o.pxS = reinterpret_cast<float4*>(opt(L.pxS));
    o.pxR = reinterpret_cast<float4*>(opt(L.pxR));
    o.pxK = reinterpret_cast<float2*>(opt(L.pxK));
    o.pxKR = reinterpret_cast<float2*>(opt(L.pxKR));
    o.pxE = reinterpret_cast<int32_t*>(opt(L.pxE));
    o.pxL = reinterpret_cast<int32_t*>(opt(L.pxL));
    return o;
}

dism::PathArgs path(const Layout& L, void* ws, int64_t B, int64_t N, int64_t H,
                    const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                    const int32_t* boundary, int32_t strip, const float* lut,
                    int64_t lut_stride) {
    dism::PathArgs a{};
    a.B = (int)B;
    a.H = (int)H;
    a.n = (int)N;
    a.iq = iq;
    a.ik = ik;
    a.hard = hard;
    a.lut = lut;
    a.lut_stride = lut_stride;
    a.bound = boundary;
    a.strip = boundary ? strip : 1;
    a.o = orders(L, ws);
    a.pnb = at<int32_t>(ws, L.pnb);
    a.prow = at<float>(ws, L.prow);
    a.prow_stride = L.prow_stride;
    return a;
}

int32_t check_common(const void* sq, const void* sk, const void* v, int32_t dtype,
                     const int32_t* iq, const int32_t* ik, int64_t B, int64_t N, int64_t H,
                     int32_t R, int32_t DV, const void* ws, int64_t ws_bytes, const char* what) {
    if (int32_t st = layout_guard()) return st;
    if (!sq || !sk || !v || !iq || !ik || !ws)
        return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (!dims_ok(B, N, H)) return fail(DISM_ERR_INVALID, "%s: positive dimensions required", what);
    if (B * H * N > INT_MAX)
        return fail(DISM_ERR_INVALID, "%s: B*H*N must be below 2^31", what);
    if (!rdv_ok(R, DV))
        return fail(DISM_ERR_UNSUPPORTED, "%s: unsupported R=%d DV=%d", what, R, DV);
    if (!dtype_ok(dtype))
        return fail(DISM_ERR_UNSUPPORTED, "%s: vector dtype must be bf16 or f32", what);
    if (!aligned16(sq) || !aligned16(sk) || !aligned16(v))
        return fail(DISM_ERR_INVALID, "%s: vector tensors must be 16-byte aligned", what);
    if (ws_bytes < layout(B, N, H, R, DV).total)
        return fail(DISM_ERR_INVALID, "%s: workspace too small", what);
    return DISM_OK;
}

// Orders, plans and dense-row data of one call (dism_hard_prepare).  cls_n > 0: the
// dense-row classification counts only each row's first cls_n positions (a prefill's rows are
// padded after the real tokens); wlo: the query resets the dense rows' boundaries follow.
int32_t prepare_impl(const void* sq, const void* sk, const void* v, int32_t dtype,
                     const int32_t* iq, const int32_t* ik, int64_t B, int64_t N, int64_t H,
                     int32_t R, int32_t DV, void* workspace, int64_t workspace_bytes,
                     int64_t cls_n, const int32_t* wlo, void* stream) {
    int32_t st = check_common(sq, sk, v, dtype, iq, ik, B, N, H, R, DV, workspace,
                              workspace_bytes, "hard prepare");
    if (st) return st;
    const Layout L = layout(B, N, H, R, DV);
    dism::SortArgs sa{};
    sa.lab[0] = iq;
    sa.lab[1] = ik;
    sa.BH = B * H;
    sa.n = (int)N;
    sa.cls_n = (int)cls_n;
    sa.prefix = wlo == nullptr ? 1 : 0;
    for (int t = 0; t < 3; ++t) sa.tmp[t] = at<int32_t>(workspace, L.tmp[t]);
    sa.o = orders(L, workspace);
    sa.pnb = at<int32_t>(workspace, L.pnb);
    dism::PathArgs pa = path(L, workspace, B, N, H, iq, ik, nullptr, nullptr, 0, nullptr, 0);
    pa.wlo = wlo;
    pa.cls_n = (int)cls_n;
    return hip_status(dism::launch_prepare(sa, pa, S(stream)), "hard prepare");
}

}  // namespace

extern "C" {

const char* dism_last_error(void) { return g_error.c_str(); }
int32_t dism_layout_check(void) {
    if (int32_t st = layout_guard()) return st;
    return ok();
}
int32_t dism_abi_version(void) { return 7; }

int32_t dism_sign_labels(const void* x, int32_t dtype, int64_t B, int64_t N, int64_t H, int32_t d,
                         int32_t* labels, void* stream) {
    if (!x || !labels) return fail(DISM_ERR_INVALID, "sign labels: null pointer");
    if (B <= 0 || N <= 0 || H <= 0 || B * N * H > ((int64_t)1 << 40))
        return fail(DISM_ERR_INVALID, "sign labels: positive dimensions required");
    if (d < 1 || d > 30) return fail(DISM_ERR_INVALID, "sign labels: symbol width must be in [1,30]");
    if (!dtype_ok(dtype)) return fail(DISM_ERR_UNSUPPORTED, "sign labels: dtype must be bf16 or f32");
    return hip_status(dism::launch_sign_labels(x, dtype, B, N, H, d, labels, S(stream)),
                      "sign labels");
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
    if (B <= 0 || H <= 0 || N <= 0 || N > INT_MAX / 2 || B * H > 65535)
        return fail(DISM_ERR_INVALID, "positive dimensions required");
    if ((N - 1) / 32 == 0) return ok();
    return hip_status(dism::launch_boundary(iq, ik, hard, B * H, (int)N, 32, 0, 1, summary,
                                            S(stream)), "hard summary");
}

int32_t dism_hard_chunk(const int32_t* summary, int32_t* boundary, int64_t BH, int64_t N,
                        void* stream) {
    if (!summary || !boundary) return fail(DISM_ERR_INVALID, "hard chunk: null pointer");
    if (BH <= 0 || BH > 65535 || N <= 0 || N > INT_MAX / 2)
        return fail(DISM_ERR_INVALID, "invalid fixed batch/head count");
    int64_t C = (N - 1) / 32;
    if (C == 0) return ok();
    return hip_status(dism::launch_chunk(summary, boundary, BH, C, (int)N, S(stream)), "hard chunk");
}

int32_t dism_hard_boundary(const int32_t* iq, const int32_t* ik, const uint8_t* hard, int64_t B,
                           int64_t H, int64_t N, int32_t strip, int32_t fill_all,
                           int32_t* boundary, void* stream) {
    if (!iq || !ik || !hard || !boundary)
        return fail(DISM_ERR_INVALID, "hard boundary: null pointer");
    if (B <= 0 || H <= 0 || N <= 0 || N > INT_MAX / 2 || B * H > 65535)
        return fail(DISM_ERR_INVALID, "positive dimensions required");
    if (strip < 1) return fail(DISM_ERR_INVALID, "boundary strip height must be positive");
    if ((N - 1) / strip == 0) return ok();
    return hip_status(dism::launch_boundary(iq, ik, hard, B * H, (int)N, strip, 1, fill_all,
                                            boundary, S(stream)), "hard boundary");
}

int64_t dism_hard_workspace_bytes(int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                  int32_t dtype) {
    if (!dims_ok(B, N, H) || B * H * N > INT_MAX || !rdv_ok(R, DV) || !dtype_ok(dtype))
        return -1;
    return layout(B, N, H, R, DV).total;
}

int32_t dism_hard_prepare(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, int64_t B, int64_t N, int64_t H,
                          int32_t R, int32_t DV, void* workspace, int64_t workspace_bytes,
                          void* stream) {
    return prepare_impl(sq, sk, v, dtype, iq, ik, B, N, H, R, DV, workspace, workspace_bytes,
                        0, nullptr, stream);
}

int32_t dism_hard_row_modes(const void* workspace, int64_t workspace_bytes, int64_t B,
                            int64_t N, int64_t H, int32_t R, int32_t DV, int32_t* modes,
                            void* stream) {
    if (!workspace || !modes) return fail(DISM_ERR_INVALID, "row modes: null pointer");
    if (!dims_ok(B, N, H) || B * H * N > INT_MAX || !rdv_ok(R, DV))
        return fail(DISM_ERR_INVALID, "row modes: invalid dimensions");
    const Layout L = layout(B, N, H, R, DV);
    if (workspace_bytes < L.total) return fail(DISM_ERR_INVALID, "row modes: workspace too small");
    return hip_status(hipMemcpyAsync(modes, static_cast<const char*>(workspace) + L.dflag,
                                     B * H * 4, hipMemcpyDeviceToDevice, S(stream)),
                      "row modes");
}

int32_t dism_hard_readout(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                          const int32_t* boundary, int32_t strip, const float* lut,
                          int64_t lut_stride, int64_t B, int64_t N, int64_t H, int32_t R,
                          int32_t DV, void* workspace, int64_t workspace_bytes, void* out,
                          int32_t out_dtype, float* lse2, int32_t* lmax, int32_t* jarg,
                          void* stream) {
    int32_t st = check_common(sq, sk, v, dtype, iq, ik, B, N, H, R, DV, workspace,
                              workspace_bytes, "hard readout");
    if (st) return st;
    if (!hard || !lut || !out || !lse2) return fail(DISM_ERR_INVALID, "hard readout: null pointer");
    if (!dtype_ok(out_dtype))
        return fail(DISM_ERR_UNSUPPORTED, "hard readout: output dtype must be bf16 or f32");
    if (lut_stride < N + 1) return fail(DISM_ERR_INVALID, "hard log-weight table is too short");
    if (boundary && strip < 1) return fail(DISM_ERR_INVALID, "invalid hard boundary strip");
    if (!aligned16(out)) return fail(DISM_ERR_INVALID, "hard readout: output must be 16-byte aligned");
    const Layout L = layout(B, N, H, R, DV);
    dism::PathArgs a = path(L, workspace, B, N, H, iq, ik, hard, boundary, strip, lut, lut_stride);
    a.sq = sq;
    a.sk = sk;
    a.v = v;
    a.out = out;
    a.out_dtype = out_dtype;
    a.lse2 = lse2;
    a.lmax = lmax;
    a.jarg = jarg;
    int32_t st2;
    if ((st2 = hip_status(dism::launch_scan_forward(a, R, DV, dtype, S(stream)), "hard readout")))
        return st2;
    if ((st2 = hip_status(dism::launch_pairs_finish(a, R, DV, dtype, S(stream)),
                          "hard readout pairs")))
        return st2;
    if ((st2 = hip_status(dism::launch_dense_forward(a, R, DV, dtype, S(stream)),
                          "hard readout dense rows")))
        return st2;
    if ((st2 = hip_status(dism::launch_level_forward(a, R, DV, dtype, S(stream)),
                          "hard readout level rows")))
        return st2;
    return hip_status(dism::launch_prefix_forward(a, R, DV, dtype, S(stream)),
                      "hard readout prefix rows");
}

int32_t dism_hard_forward(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                          const int32_t* boundary, int32_t strip, const float* lut,
                          int64_t lut_stride, int64_t B, int64_t N, int64_t H, int32_t R,
                          int32_t DV, void* workspace, int64_t workspace_bytes, void* out,
                          int32_t out_dtype, float* lse2, int32_t* lmax, int32_t* jarg,
                          void* stream) {
    int32_t st = check_common(sq, sk, v, dtype, iq, ik, B, N, H, R, DV, workspace,
                              workspace_bytes, "hard forward");
    if (st) return st;
    if (!hard || !lut || !out || !lse2) return fail(DISM_ERR_INVALID, "hard forward: null pointer");
    if (!dtype_ok(out_dtype))
        return fail(DISM_ERR_UNSUPPORTED, "hard forward: output dtype must be bf16 or f32");
    if (lut_stride < N + 1) return fail(DISM_ERR_INVALID, "hard log-weight table is too short");
    if (boundary && strip < 1) return fail(DISM_ERR_INVALID, "invalid hard boundary strip");
    if (!aligned16(out)) return fail(DISM_ERR_INVALID, "hard forward: output must be 16-byte aligned");
    const Layout L = layout(B, N, H, R, DV);
    dism::SortArgs sa{};
    sa.lab[0] = iq;
    sa.lab[1] = ik;
    sa.BH = B * H;
    sa.n = (int)N;
    for (int t = 0; t < 3; ++t) sa.tmp[t] = at<int32_t>(workspace, L.tmp[t]);
    sa.o = orders(L, workspace);
    sa.pnb = at<int32_t>(workspace, L.pnb);
    sa.prefix = 1;
    dism::PathArgs a = path(L, workspace, B, N, H, iq, ik, hard, boundary, strip, lut, lut_stride);
    a.sq = sq;
    a.sk = sk;
    a.v = v;
    a.out = out;
    a.out_dtype = out_dtype;
    a.lse2 = lse2;
    a.lmax = lmax;
    a.jarg = jarg;
    // The label order (what the length-1 scan needs) and the bigram half of the prepare (what
    // only the pair kernels need) are independent: the bigram half runs on a side stream while
    // the scan takes the rows prepared in LDS, counting their bigram partners itself (phase
    // 1); after the join the scan takes the remaining rows from the plan's counts (phase 2),
    // then the pair kernels run.  Without a side stream the same launches run in order.
    // The row flags (classification) are read by the bigram half and by the scan, not by
    // the label order: with a side stream they are computed there, first, concurrently with
    // the label order, and the caller's stream waits for them just before the scan.
    const hipStream_t s = S(stream);
    SideLease lease;
    SideStream* side = lease.get();
    hipStream_t ps = s;
    if (side) {
        if (hipEventRecord(side->fork, s) != hipSuccess ||
            hipStreamWaitEvent(side->stream, side->fork, 0) != hipSuccess)
            side = nullptr;
        else
            ps = side->stream;
    }
    hipError_t e = dism::launch_classify(sa, ps);
    bool classified = true;
    if (e == hipSuccess && side) classified = hipEventRecord(side->mid, ps) == hipSuccess;
    if (e == hipSuccess) e = dism::launch_prepare_labels(sa, a, s);
    if (e == hipSuccess && side && classified)
        classified = hipStreamWaitEvent(s, side->mid, 0) == hipSuccess;
    if (e == hipSuccess && !classified) e = hipErrorUnknown;
    if (e == hipSuccess) e = dism::launch_prepare_pairs(sa, a, ps);
    // rows of the pairless modes (dense tiles, level rows, prefix rows) read neither the
    // scan's records nor the pair plan: their readouts follow the prepare on the side stream,
    // off the scan -> pair-correction chain (their launches exit at once without such rows)
    if (e == hipSuccess) e = dism::launch_dense_forward(a, R, DV, dtype, ps);
    if (e == hipSuccess) e = dism::launch_level_forward(a, R, DV, dtype, ps);
    if (e == hipSuccess) e = dism::launch_prefix_forward(a, R, DV, dtype, ps);
    if (e == hipSuccess) {
        a.fwd_phase = 1;
        e = dism::launch_scan_forward(a, R, DV, dtype, s);
    }
    bool joined = true;
    if (side)  // join even after an error, so the caller's stream never runs ahead
        joined = hipEventRecord(side->join, side->stream) == hipSuccess &&
                 hipStreamWaitEvent(s, side->join, 0) == hipSuccess;
    if ((st = hip_status(e, "hard forward"))) return st;
    if (!joined) return fail(DISM_ERR_HIP, "hard forward: stream join failed");
    a.fwd_phase = 2;
    if ((st = hip_status(dism::launch_scan_forward(a, R, DV, dtype, s), "hard forward")))
        return st;
    return hip_status(dism::launch_pairs_finish(a, R, DV, dtype, s), "hard forward pairs");
}

}  // extern "C"

// ---------------------------------------------------------------------------------------
// Allocation-free forward: the workspace is this file-scope device array instead of a caller
// buffer.  Each device the library runs on holds its own copy until the process ends.  In
// host code `scratch` only names the symbol: its device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only that address is
// passed to kernels.
constexpr int64_t NOALLOC_SCRATCH_BYTES = int64_t(256) << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mutex;
void* g_scratch_ptr[MAX_DEVICES] = {};

// device address of `scratch` on the current device (null after an error, with its text set)
void* scratch_address() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        fail(DISM_ERR_HIP, "forward (no allocation): no current HIP device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            fail(DISM_ERR_HIP, "forward (no allocation): hipGetSymbolAddress failed: %d (%s)",
                 (int)e, hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}
}  // namespace

extern "C" {

int64_t dism_hard_forward_noalloc_max_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

int32_t dism_hard_forward_noalloc(const void* sq, const void* sk, const void* v, int32_t dtype,
                                  const int32_t* iq, const int32_t* ik, const uint8_t* hard,
                                  const float* lut, int64_t lut_stride, int64_t B, int64_t N,
                                  int64_t H, int32_t R, int32_t DV, void* out, int32_t out_dtype,
                                  float* lse2, int32_t* lmax, int32_t* jarg, void* stream) {
    const char* what = "hard forward (no allocation)";
    if (int32_t lg = layout_guard()) return lg;
    if (!dims_ok(B, N, H) || B * H * N > INT_MAX || !rdv_ok(R, DV) || !dtype_ok(dtype))
        return fail(DISM_ERR_INVALID, "%s: unsupported dimensions or dtype", what);
    const int64_t need = layout(B, N, H, R, DV).total;
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(DISM_ERR_INVALID,
                    "%s: this shape needs %lld workspace bytes, above the %lld of the library's "
                    "device scratch; use dism_hard_forward with a caller workspace",
                    what, (long long)need, (long long)NOALLOC_SCRATCH_BYTES);
    void* ws = scratch_address();
    if (!ws) return DISM_ERR_HIP;
    // the staged forward on the caller's stream only: prepare, then the readout (label scans,
    // bigram corrections, dense rows); no side stream, no allocation
    int32_t st = prepare_impl(sq, sk, v, dtype, iq, ik, B, N, H, R, DV, ws, need, 0, nullptr,
                              stream);
    if (st) return st;
    return dism_hard_readout(sq, sk, v, dtype, iq, ik, hard, nullptr, 0, lut, lut_stride, B, N,
                             H, R, DV, ws, need, out, out_dtype, lse2, lmax, jarg, stream);
}

}  // extern "C"

static int32_t backward_common(const void* sq, const void* sk, const void* v, const void* dout,
                               int32_t dtype, const int32_t* iq, const int32_t* ik,
                               const uint8_t* hard, const int32_t* boundary, int32_t strip,
                               const float* lut, int64_t lut_stride, const float* lse2,
                               int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                               void* workspace, int64_t workspace_bytes, dism::PathArgs* a,
                               const char* what) {
    int32_t st = check_common(sq, sk, v, dtype, iq, ik, B, N, H, R, DV, workspace,
                              workspace_bytes, what);
    if (st) return st;
    if (!dout || !hard || !lut || !lse2) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (lut_stride < N + 1) return fail(DISM_ERR_INVALID, "hard log-weight table is too short");
    if (boundary && strip < 1) return fail(DISM_ERR_INVALID, "invalid hard boundary strip");
    if (!aligned16(dout)) return fail(DISM_ERR_INVALID, "%s: dO must be 16-byte aligned", what);
    const Layout L = layout(B, N, H, R, DV);
    *a = path(L, workspace, B, N, H, iq, ik, hard, boundary, strip, lut, lut_stride);
    a->sq = sq;
    a->sk = sk;
    a->v = v;
    a->dout = dout;
    a->lse2 = const_cast<float*>(lse2);
    return DISM_OK;
}

extern "C" {

int32_t dism_hard_backward_row_pairs(const void* sq, const void* sk, const void* v,
                                     const void* dout, int32_t dtype, const int32_t* iq,
                                     const int32_t* ik, const uint8_t* hard,
                                     const int32_t* boundary, int32_t strip, const float* lut,
                                     const float* dlut, int64_t lut_stride, const float* lse2,
                                     int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
    dism::PathArgs a{};
    int32_t st = backward_common(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip, lut,
                                 lut_stride, lse2, B, N, H, R, DV, workspace, workspace_bytes,
                                 &a, "hard backward row pairs");
    if (st) return st;
    if (!dlut) return fail(DISM_ERR_INVALID, "hard backward: null pointer");
    a.dlut = dlut;
    return hip_status(dism::launch_pairs_rows(a, R, DV, dtype, S(stream)),
                      "hard backward row pairs");
}

int32_t dism_hard_backward_queries(const void* sq, const void* sk, const void* v,
                                   const void* dout, int32_t dtype, const int32_t* iq,
                                   const int32_t* ik, const uint8_t* hard,
                                   const int32_t* boundary, int32_t strip, const float* lut,
                                   const float* dlut, int64_t lut_stride, const float* lse2,
                                   int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                   void* workspace, int64_t workspace_bytes, float* dsq,
                                   float* rowtau, void* stream) {
    dism::PathArgs a{};
    int32_t st = backward_common(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip, lut,
                                 lut_stride, lse2, B, N, H, R, DV, workspace, workspace_bytes,
                                 &a, "hard backward queries");
    if (st) return st;
    if (!dlut || !dsq || !rowtau) return fail(DISM_ERR_INVALID, "hard backward: null pointer");
    a.dlut = dlut;
    a.dsq = dsq;
    a.rowtau = rowtau;
    // the dense, level and prefix rows (disjoint from the scan's rows) beside the label scan
    PairlessFork fork(S(stream));
    if ((st = hip_status(dism::launch_dense_rows(a, R, DV, dtype, fork.side()),
                         "hard backward dense rows")) ||
        (st = hip_status(dism::launch_level_rows(a, R, DV, dtype, fork.side()),
                         "hard backward level rows")) ||
        (st = hip_status(dism::launch_prefix_rows(a, R, DV, dtype, fork.side()),
                         "hard backward prefix rows")) ||
        (st = hip_status(dism::launch_scan_rows(a, R, DV, dtype, S(stream)),
                         "hard backward rows")))
        fork.join();
    else
        st = fork.join() ? DISM_OK : fail(DISM_ERR_HIP, "hard backward rows: stream join failed");
    return st;
}

int32_t dism_hard_backward_keys(const void* sq, const void* sk, const void* v, const void* dout,
                                int32_t dtype, const int32_t* iq, const int32_t* ik,
                                const uint8_t* hard, const int32_t* boundary, int32_t strip,
                                const float* lut, int64_t lut_stride, const float* lse2,
                                int64_t B, int64_t N, int64_t H, int32_t R, int32_t DV,
                                void* workspace, int64_t workspace_bytes, float* dsk, float* dv,
                                void* stream) {
    dism::PathArgs a{};
    int32_t st = backward_common(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip, lut,
                                 lut_stride, lse2, B, N, H, R, DV, workspace, workspace_bytes,
                                 &a, "hard backward keys");
    if (st) return st;
    if (!dsk || !dv) return fail(DISM_ERR_INVALID, "hard backward: null pointer");
    a.dsk = dsk;
    a.dv = dv;
    // the dense, level and prefix rows' keys (disjoint from the scan's rows) beside the scan
    PairlessFork fork(S(stream));
    if ((st = hip_status(dism::launch_dense_keys(a, R, DV, dtype, fork.side()),
                         "hard backward dense keys")) ||
        (st = hip_status(dism::launch_level_keys(a, R, DV, dtype, fork.side()),
                         "hard backward level keys")) ||
        (st = hip_status(dism::launch_prefix_keys(a, R, DV, dtype, fork.side()),
                         "hard backward prefix keys")) ||
        (st = hip_status(dism::launch_scan_keys(a, R, DV, dtype, S(stream)),
                         "hard backward keys")))
        fork.join();
    else
        st = fork.join() ? DISM_OK : fail(DISM_ERR_HIP, "hard backward keys: stream join failed");
    return st;
}

int32_t dism_hard_backward_key_pairs(const void* sq, const void* sk, const void* v,
                                     const void* dout, int32_t dtype, const int32_t* iq,
                                     const int32_t* ik, const uint8_t* hard,
                                     const int32_t* boundary, int32_t strip, const float* lut,
                                     int64_t lut_stride, const float* lse2, int64_t B, int64_t N,
                                     int64_t H, int32_t R, int32_t DV, void* workspace,
                                     int64_t workspace_bytes, float* dsk, float* dv,
                                     void* stream) {
    dism::PathArgs a{};
    int32_t st = backward_common(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip, lut,
                                 lut_stride, lse2, B, N, H, R, DV, workspace, workspace_bytes,
                                 &a, "hard backward key pairs");
    if (st) return st;
    if (!dsk || !dv) return fail(DISM_ERR_INVALID, "hard backward: null pointer");
    a.dsk = dsk;
    a.dv = dv;
    return hip_status(dism::launch_pairs_keys(a, R, DV, dtype, S(stream)),
                      "hard backward key pairs");
}

int32_t dism_hard_tau_reduce(const float* rowtau, int64_t B, int64_t H, int64_t N, float* dtau,
                             void* stream) {
    if (!rowtau || !dtau) return fail(DISM_ERR_INVALID, "tau reduce: null pointer");
    if (B <= 0 || H <= 0 || N <= 0 || H > 65535)
        return fail(DISM_ERR_INVALID, "positive dimensions required");
    return hip_status(dism::launch_tau_reduce(rowtau, (int)B, (int)H, N, dtau, S(stream)),
                      "hard tau reduce");
}

int32_t dism_hard_backward(const void* sq, const void* sk, const void* v, const void* dout,
                           int32_t dtype, const int32_t* iq, const int32_t* ik,
                           const uint8_t* hard, const int32_t* boundary, int32_t strip,
                           const float* lut, const float* dlut, int64_t lut_stride,
                           const float* lse2, int64_t B, int64_t N, int64_t H, int32_t R,
                           int32_t DV, void* workspace, int64_t workspace_bytes, float* dsq,
                           float* dsk, float* dv, float* rowtau, float* dtau, void* stream) {
    if (!dtau) return fail(DISM_ERR_INVALID, "hard backward: null pointer");
    // the key chain (keys -> key pairs) and the query-row chain (row pairs -> queries -> tau)
    // are independent: the key chain runs on a side stream, forked from and joined back into
    // the caller's stream (the row pairs are enqueued first so their persistent grid starts
    // first)
    SideLease lease;
    SideStream* side = lease.get();
    const hipStream_t s = S(stream);
    void* ks = stream;
    if (side) {
        if (hipEventRecord(side->fork, s) != hipSuccess ||
            hipStreamWaitEvent(side->stream, side->fork, 0) != hipSuccess)
            side = nullptr;
        else
            ks = side->stream;
    }
    int32_t st = dism_hard_backward_row_pairs(sq, sk, v, dout, dtype, iq, ik, hard, boundary,
                                              strip, lut, dlut, lut_stride, lse2, B, N, H, R, DV,
                                              workspace, workspace_bytes, stream);
    if (!st)
        st = dism_hard_backward_keys(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip,
                                     lut, lut_stride, lse2, B, N, H, R, DV, workspace,
                                     workspace_bytes, dsk, dv, ks);
    if (!st)
        st = dism_hard_backward_key_pairs(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip,
                                          lut, lut_stride, lse2, B, N, H, R, DV, workspace,
                                          workspace_bytes, dsk, dv, ks);
    if (!st)
        st = dism_hard_backward_queries(sq, sk, v, dout, dtype, iq, ik, hard, boundary, strip,
                                        lut, dlut, lut_stride, lse2, B, N, H, R, DV, workspace,
                                        workspace_bytes, dsq, rowtau, stream);
    if (!st) st = dism_hard_tau_reduce(rowtau, B, H, N, dtau, stream);
    if (side) {  // join even after an error, so the caller's stream never runs ahead
        const bool joined = hipEventRecord(side->join, side->stream) == hipSuccess &&
                            hipStreamWaitEvent(s, side->join, 0) == hipSuccess;
        if (!st && !joined) return fail(DISM_ERR_HIP, "hard backward: stream join failed");
    }
    return st;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------
// Packed (varlen) batch-1 layouts: the fixed-length workspace of (B = 1, N, H) followed by the
// document-tagged labels, the document start of every token and all-ones row flags
// (dism_packed.hip).
namespace {

struct PackedLayout {
    Layout base;
    int64_t tq, tk, dstart, dindex, ones, total;
};

PackedLayout packed_layout(int64_t N, int64_t H, int32_t R, int32_t DV) {
    PackedLayout P;
    P.base = layout(1, N, H, R, DV);
    int64_t o = P.base.total;
    P.tq = o;
    o += align256(H * N * 4);
    P.tk = o;
    o += align256(H * N * 4);
    P.dstart = o;
    o += align256(N * 4);
    P.dindex = o;
    o += align256(N * 4);
    P.ones = o;
    o += align256(H);
    P.total = o;
    return P;
}

int32_t check_packed(const void* sq, const void* sk, const void* v, int32_t dtype, int64_t N,
                     int64_t H, int32_t R, int32_t DV, const void* ws, int64_t ws_bytes,
                     const char* what) {
    if (!sq || !sk || !v || !ws) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (!dims_ok(1, N, H)) return fail(DISM_ERR_INVALID, "%s: positive dimensions required", what);
    if (H * N > INT_MAX) return fail(DISM_ERR_INVALID, "%s: H*N must be below 2^31", what);
    if (!rdv_ok(R, DV))
        return fail(DISM_ERR_UNSUPPORTED, "%s: unsupported R=%d DV=%d", what, R, DV);
    if (!dtype_ok(dtype))
        return fail(DISM_ERR_UNSUPPORTED, "%s: vector dtype must be bf16 or f32", what);
    if (!aligned16(sq) || !aligned16(sk) || !aligned16(v))
        return fail(DISM_ERR_INVALID, "%s: vector tensors must be 16-byte aligned", what);
    if (ws_bytes < packed_layout(N, H, R, DV).total)
        return fail(DISM_ERR_INVALID, "%s: workspace too small", what);
    return DISM_OK;
}

int32_t check_rows(const uint8_t* hard, int64_t rows, int64_t N, const float* lut,
                   int64_t lut_stride, int64_t max_length, const char* what) {
    if (!hard || !lut) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (rows <= 0 || N % rows != 0 || (N / rows) % 256 != 0)
        return fail(DISM_ERR_INVALID,
                    "packed hard rows must evenly divide tokens into 256-aligned training rows");
    if (max_length <= 0 || max_length > N)
        return fail(DISM_ERR_INVALID, "%s: invalid longest document length", what);
    if (lut_stride < max_length + 1)
        return fail(DISM_ERR_INVALID, "hard log-weight table is too short");
    return DISM_OK;
}

dism::PathArgs packed_path(const PackedLayout& P, void* ws, int64_t N, int64_t H,
                           const float* lut, int64_t lut_stride) {
    dism::PathArgs a = path(P.base, ws, 1, N, H, at<int32_t>(ws, P.tq), at<int32_t>(ws, P.tk),
                            at<uint8_t>(ws, P.ones), nullptr, 0, lut, lut_stride);
    a.dstart = at<int32_t>(ws, P.dstart);
    return a;
}

dism::PackedZero packed_zero(const uint8_t* hard, int64_t rows, int64_t N, int64_t H, int32_t R,
                             int32_t DV) {
    dism::PackedZero z{};
    z.hard = hard;
    z.row_tokens = N / rows;
    z.H = H;
    z.n = N;
    z.R = R;
    z.DV = DV;
    return z;
}

}  // namespace

extern "C" {

int64_t dism_hard_packed_workspace_bytes(int64_t N, int64_t H, int32_t R, int32_t DV,
                                         int32_t dtype) {
    if (!dims_ok(1, N, H) || H * N > INT_MAX || !rdv_ok(R, DV) || !dtype_ok(dtype)) return -1;
    return packed_layout(N, H, R, DV).total;
}

int32_t dism_hard_packed_prepare(const void* sq, const void* sk, const void* v, int32_t dtype,
                                 const int32_t* iq, const int32_t* ik,
                                 const int32_t* cu_seqlens, int64_t docs, int64_t N, int64_t H,
                                 int32_t R, int32_t DV, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
    const char* what = "packed hard prepare";
    if (int32_t lg = layout_guard()) return lg;
    int32_t st = check_packed(sq, sk, v, dtype, N, H, R, DV, workspace, workspace_bytes, what);
    if (st) return st;
    if (!iq || !ik || !cu_seqlens) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (docs <= 0 || docs > N) return fail(DISM_ERR_INVALID, "%s: invalid document count", what);
    if (2 * N * docs > ((int64_t)1 << 32))
        return fail(DISM_ERR_INVALID, "%s: 2 * N * documents must not exceed 2^32", what);
    const PackedLayout P = packed_layout(N, H, R, DV);
    int32_t* tq = at<int32_t>(workspace, P.tq);
    int32_t* tk = at<int32_t>(workspace, P.tk);
    int32_t* dindex = at<int32_t>(workspace, P.dindex);
    hipStream_t s = S(stream);
    // document of every token, then dense label ranks from a label sort of the raw labels
    dism::SortArgs raw{};
    raw.lab[0] = iq;
    raw.lab[1] = ik;
    raw.BH = H;
    raw.n = (int)N;
    for (int t = 0; t < 3; ++t) raw.tmp[t] = at<int32_t>(workspace, P.base.tmp[t]);
    raw.o = orders(P.base, workspace);
    raw.pnb = at<int32_t>(workspace, P.base.pnb);
    if ((st = hip_status(dism::launch_packed_docs(cu_seqlens, (int)docs, H, N,
                                                  at<int32_t>(workspace, P.dstart), dindex,
                                                  at<uint8_t>(workspace, P.ones), s), what)) ||
        (st = hip_status(dism::launch_sort_labels(raw, s), what)) ||
        (st = hip_status(dism::launch_packed_tags(raw.o.corder, raw.o.clab, dindex, (int)docs, H,
                                                  N, tq, tk, s), what)))
        return st;
    dism::SortArgs sa{};
    sa.lab[0] = tq;
    sa.lab[1] = tk;
    sa.BH = H;
    sa.n = (int)N;
    for (int t = 0; t < 3; ++t) sa.tmp[t] = at<int32_t>(workspace, P.base.tmp[t]);
    sa.o = orders(P.base, workspace);
    sa.pnb = at<int32_t>(workspace, P.base.pnb);
    const dism::PathArgs pa = packed_path(P, workspace, N, H, nullptr, 0);
    return hip_status(dism::launch_prepare(sa, pa, s), what);
}

int32_t dism_hard_packed_readout(const void* sq, const void* sk, const void* v, int32_t dtype,
                                 const uint8_t* hard, int64_t rows, const float* lut,
                                 int64_t lut_stride, int64_t max_length, int64_t N, int64_t H,
                                 int32_t R, int32_t DV, void* workspace, int64_t workspace_bytes,
                                 void* out, int32_t out_dtype, float* lse2, int32_t* lmax,
                                 int32_t* jarg, void* stream) {
    const char* what = "packed hard readout";
    if (int32_t lg = layout_guard()) return lg;
    int32_t st = check_packed(sq, sk, v, dtype, N, H, R, DV, workspace, workspace_bytes, what);
    if (st) return st;
    if ((st = check_rows(hard, rows, N, lut, lut_stride, max_length, what))) return st;
    if (!out || !lse2) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (!dtype_ok(out_dtype))
        return fail(DISM_ERR_UNSUPPORTED, "%s: output dtype must be bf16 or f32", what);
    if (!aligned16(out)) return fail(DISM_ERR_INVALID, "%s: output must be 16-byte aligned", what);
    const PackedLayout P = packed_layout(N, H, R, DV);
    dism::PathArgs a = packed_path(P, workspace, N, H, lut, lut_stride);
    a.sq = sq;
    a.sk = sk;
    a.v = v;
    a.out = out;
    a.out_dtype = out_dtype;
    a.lse2 = lse2;
    a.lmax = lmax;
    a.jarg = jarg;
    if ((st = hip_status(dism::launch_scan_forward(a, R, DV, dtype, S(stream)), what))) return st;
    if ((st = hip_status(dism::launch_pairs_finish(a, R, DV, dtype, S(stream)), what))) return st;
    if ((st = hip_status(dism::launch_dense_forward(a, R, DV, dtype, S(stream)), what))) return st;
    dism::PackedZero z = packed_zero(hard, rows, N, H, R, DV);
    z.out = out;
    z.out_dtype = out_dtype;
    z.lse2 = lse2;
    z.lmax = lmax;
    z.jarg = jarg;
    return hip_status(dism::launch_packed_soft_zero(z, S(stream)), what);
}

int32_t dism_hard_packed_backward(const void* sq, const void* sk, const void* v,
                                  const void* dout, int32_t dtype, const uint8_t* hard,
                                  int64_t rows, const float* lut, const float* dlut,
                                  int64_t lut_stride, int64_t max_length, const float* lse2,
                                  int64_t N, int64_t H, int32_t R, int32_t DV, void* workspace,
                                  int64_t workspace_bytes, float* dsq, float* dsk, float* dv,
                                  float* rowtau, float* dtau, void* stream) {
    const char* what = "packed hard backward";
    if (int32_t lg = layout_guard()) return lg;
    int32_t st = check_packed(sq, sk, v, dtype, N, H, R, DV, workspace, workspace_bytes, what);
    if (st) return st;
    if ((st = check_rows(hard, rows, N, lut, lut_stride, max_length, what))) return st;
    if (!dout || !dlut || !lse2 || !dsq || !dsk || !dv || !rowtau || !dtau)
        return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (!aligned16(dout)) return fail(DISM_ERR_INVALID, "%s: dO must be 16-byte aligned", what);
    const PackedLayout P = packed_layout(N, H, R, DV);
    dism::PathArgs a = packed_path(P, workspace, N, H, lut, lut_stride);
    a.sq = sq;
    a.sk = sk;
    a.v = v;
    a.dout = dout;
    a.dlut = dlut;
    a.lse2 = const_cast<float*>(lse2);
    a.dsq = dsq;
    a.dsk = dsk;
    a.dv = dv;
    a.rowtau = rowtau;
    hipStream_t s = S(stream);
    if ((st = hip_status(dism::launch_pairs_rows(a, R, DV, dtype, s), what))) return st;
    if ((st = hip_status(dism::launch_scan_rows(a, R, DV, dtype, s), what))) return st;
    if ((st = hip_status(dism::launch_scan_keys(a, R, DV, dtype, s), what))) return st;
    if ((st = hip_status(dism::launch_pairs_keys(a, R, DV, dtype, s), what))) return st;
    if ((st = hip_status(dism::launch_dense_rows(a, R, DV, dtype, s), what))) return st;
    if ((st = hip_status(dism::launch_dense_keys(a, R, DV, dtype, s), what))) return st;
    dism::PackedZero z = packed_zero(hard, rows, N, H, R, DV);
    z.dsq = dsq;
    z.dsk = dsk;
    z.dv = dv;
    z.rowtau = rowtau;
    if ((st = hip_status(dism::launch_packed_soft_zero(z, s), what))) return st;
    return hip_status(dism::launch_tau_reduce(rowtau, 1, (int)H, N, dtau, s), what);
}

}  // extern "C"

// ---------------------------------------------------------------------------------------
// Inference: prefill with query resets, and the incremental decoder (dism_decode.hip).
namespace {

struct DecoderLayout {
    int64_t meta, qlab, klab, skh, vh, slot_label, slot_cnt, slot_last, M, slot_blocks, pool,
        scratch, total;
    int bcap, pool_blocks;
};

bool decoder_dims_ok(int64_t rows, int32_t R, int32_t DV, int64_t cap, int32_t slots,
                     int32_t dtype) {
    return rows > 0 && rows <= 65535 && rdv_ok(R, DV) && dtype_ok(dtype) && cap > 0 &&
           cap <= (1 << 24) && slots >= 64 && slots <= (1 << 20) && (slots & (slots - 1)) == 0;
}

DecoderLayout decoder_layout(int64_t rows, int32_t R, int32_t DV, int64_t cap, int32_t slots,
                             int32_t dtype) {
    DecoderLayout D;
    const int64_t esz = dtype == DISM_BF16 ? 2 : 4;
    D.bcap = (int)((cap + dism::LIST_BLOCK - 1) / dism::LIST_BLOCK);
    D.pool_blocks = D.bcap + slots;
    int64_t o = 0;
    auto take = [&](int64_t bytes) {
        int64_t a = o;
        o += align256(bytes);
        return a;
    };
    D.meta = take(rows * 4 * 4);
    D.qlab = take(rows * cap * 4);
    D.klab = take(rows * cap * 4);
    D.skh = take(rows * cap * R * esz);
    D.vh = take(rows * cap * DV * esz);
    D.slot_label = take(rows * slots * 4);
    D.slot_cnt = take(rows * slots * 4);
    D.slot_last = take(rows * slots * 4);
    D.M = take(rows * slots * (int64_t)R * DV * 4);
    D.slot_blocks = take(rows * slots * (int64_t)D.bcap * 4);
    D.pool = take(rows * (int64_t)D.pool_blocks * dism::LIST_BLOCK * 4);
    D.scratch = take(rows * cap * 4);
    D.total = o;
    return D;
}

dism::DecodeArgs decode_args(void* state, const DecoderLayout& D, int64_t rows, int64_t H,
                             int32_t R, int32_t DV, int64_t capacity, int32_t slots) {
    dism::DecodeArgs a{};
    a.rows = (int)rows;
    a.H = (int)H;
    a.cap = (int)capacity;
    a.slots = slots;
    a.bcap = D.bcap;
    a.R = R;
    a.DV = DV;
    a.meta = at<int32_t>(state, D.meta);
    a.qlab = at<int32_t>(state, D.qlab);
    a.klab = at<int32_t>(state, D.klab);
    a.skh = at<void>(state, D.skh);
    a.vh = at<void>(state, D.vh);
    a.slot_label = at<int32_t>(state, D.slot_label);
    a.slot_cnt = at<int32_t>(state, D.slot_cnt);
    a.slot_last = at<int32_t>(state, D.slot_last);
    a.M = at<float>(state, D.M);
    a.slot_blocks = at<int32_t>(state, D.slot_blocks);
    a.pool = at<int32_t>(state, D.pool);
    a.scratch = at<int32_t>(state, D.scratch);
    a.pool_blocks = D.pool_blocks;
    return a;
}

int64_t prefill_extra(int64_t B, int64_t N, int64_t H) {
    return align256(B * H) + align256(B * H * N * 4);
}

}  // namespace

extern "C" {

int64_t dism_hard_prefill_workspace_bytes(int64_t B, int64_t N, int64_t H, int32_t R,
                                          int32_t DV, int32_t dtype) {
    if (!dims_ok(B, N, H) || B * H * N > INT_MAX || !rdv_ok(R, DV) || !dtype_ok(dtype))
        return -1;
    return layout(B, N, H, R, DV).total + prefill_extra(B, N, H);
}

int32_t dism_hard_prefill(const void* sq, const void* sk, const void* v, int32_t dtype,
                          const int32_t* iq, const int32_t* ik, const uint8_t* reset,
                          const float* lut, int64_t lut_stride, int64_t B, int64_t N,
                          int64_t n_valid, int64_t H, int32_t R, int32_t DV, void* workspace,
                          int64_t workspace_bytes, float* out, float* lse2, void* stream) {
    const char* what = "hard prefill";
    if (int32_t lg = layout_guard()) return lg;
    int32_t st = check_common(sq, sk, v, dtype, iq, ik, B, N, H, R, DV, workspace,
                              workspace_bytes, what);
    if (st) return st;
    if (n_valid <= 0 || n_valid > N)
        return fail(DISM_ERR_INVALID, "%s: valid length must be in [1, N]", what);
    if (!lut || !out || !lse2) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (lut_stride < N + 1) return fail(DISM_ERR_INVALID, "hard log-weight table is too short");
    if (!aligned16(out)) return fail(DISM_ERR_INVALID, "%s: output must be 16-byte aligned", what);
    const Layout L = layout(B, N, H, R, DV);
    if (workspace_bytes < L.total + prefill_extra(B, N, H))
        return fail(DISM_ERR_INVALID, "%s: workspace too small", what);
    uint8_t* ones = at<uint8_t>(workspace, L.total);
    int32_t* wlo = at<int32_t>(workspace, L.total + align256(B * H));
    hipStream_t s = S(stream);
    // all-hard row flags (bytes of one, a fill kernel), then the reset starts
    if ((st = hip_status(dism::launch_fill_i32(reinterpret_cast<int32_t*>(ones),
                                               align256(B * H) / 4, 0x01010101, s), what)))
        return st;
    if (reset && (st = hip_status(dism::launch_reset_starts(reset, B * H, N, wlo, s), what)))
        return st;
    if ((st = prepare_impl(sq, sk, v, dtype, iq, ik, B, N, H, R, DV, workspace,
                           workspace_bytes, n_valid, reset ? wlo : nullptr, stream)))
        return st;
    dism::PathArgs a = path(L, workspace, B, N, H, iq, ik, ones, nullptr, 0, lut, lut_stride);
    a.wlo = reset ? wlo : nullptr;
    a.cls_n = (int)n_valid;  // prefix rows take their real positions only
    a.sq = sq;
    a.sk = sk;
    a.v = v;
    a.out = out;
    a.out_dtype = DISM_F32;
    a.lse2 = lse2;
    if ((st = hip_status(dism::launch_scan_forward(a, R, DV, dtype, s), what))) return st;
    if ((st = hip_status(dism::launch_pairs_finish(a, R, DV, dtype, s), what))) return st;
    if ((st = hip_status(dism::launch_dense_forward(a, R, DV, dtype, s), what))) return st;
    const hipError_t le = dism::launch_level_forward(a, R, DV, dtype, s);
    if (le != hipSuccess) return hip_status(le, what);
    return hip_status(dism::launch_prefix_forward(a, R, DV, dtype, s), what);
}

int64_t dism_decoder_state_bytes(int64_t rows, int32_t R, int32_t DV, int64_t capacity,
                                 int32_t slots, int32_t dtype) {
    if (!decoder_dims_ok(rows, R, DV, capacity, slots, dtype)) return -1;
    return decoder_layout(rows, R, DV, capacity, slots, dtype).total;
}

int32_t dism_decoder_init(void* state, int64_t state_bytes, int64_t rows, int32_t R, int32_t DV,
                          int64_t capacity, int32_t slots, int32_t dtype, void* stream) {
    const char* what = "decoder init";
    if (int32_t lg = layout_guard()) return lg;
    if (!state) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (!decoder_dims_ok(rows, R, DV, capacity, slots, dtype))
        return fail(DISM_ERR_INVALID, "%s: invalid decoder dimensions", what);
    const DecoderLayout D = decoder_layout(rows, R, DV, capacity, slots, dtype);
    if (state_bytes < D.total) return fail(DISM_ERR_INVALID, "%s: state too small", what);
    // zero every section (a fill kernel, not a memset node: safe under graph capture)
    return hip_status(dism::launch_fill_i32(static_cast<int32_t*>(state), D.total / 4, 0,
                                            S(stream)), what);
}

int32_t dism_decoder_step(void* state, int64_t state_bytes, int64_t B, int64_t H, int32_t R,
                          int32_t DV, int64_t capacity, int32_t slots, int32_t dtype, int64_t n,
                          const int32_t* iq, const int32_t* ik, const uint8_t* reset,
                          const void* sq, const void* sk, const void* v, const float* lut,
                          int64_t lut_stride, float* out, float* lse2, void* stream) {
    const char* what = "decoder step";
    if (int32_t lg = layout_guard()) return lg;
    if (!state || !iq || !ik || !sk || !v) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    const int64_t rows = B * H;
    if (B <= 0 || H <= 0 || !decoder_dims_ok(rows, R, DV, capacity, slots, dtype))
        return fail(DISM_ERR_INVALID, "%s: invalid decoder dimensions", what);
    if (n <= 0 || n > capacity) return fail(DISM_ERR_INVALID, "%s: invalid token count", what);
    if (out && (!sq || !lut)) return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (out && lut_stride < capacity + 1)
        return fail(DISM_ERR_INVALID, "hard log-weight table is too short");
    const DecoderLayout D = decoder_layout(rows, R, DV, capacity, slots, dtype);
    if (state_bytes < D.total) return fail(DISM_ERR_INVALID, "%s: state too small", what);
    dism::DecodeArgs a = decode_args(state, D, rows, H, R, DV, capacity, slots);
    a.n = (int)n;
    a.iq = iq;
    a.ik = ik;
    a.reset = reset;
    a.sq = sq;
    a.sk = sk;
    a.v = v;
    a.lut = out ? lut : nullptr;
    a.lut_stride = lut_stride;
    a.out = out;
    a.lse2 = out ? lse2 : nullptr;
    return hip_status(dism::launch_decode(a, dtype, S(stream)), what);
}

}  // extern "C"

extern "C" {

int32_t dism_vocab_labels(const void* x, const void* vocab, int64_t vocab_head_stride, int64_t B,
                          int64_t N, int64_t H, int64_t V, int32_t D, int32_t* labels,
                          int32_t* scratch, void* stream) {
    const char* what = "vocabulary labels";
    if (int32_t lg = layout_guard()) return lg;
    if (!x || !vocab || !labels || !scratch)
        return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    if (B <= 0 || N <= 0 || H <= 0 || V <= 0 || V > INT_MAX || B * H * N >= INT_MAX)
        return fail(DISM_ERR_INVALID, "%s: positive dimensions required", what);
    if (D != 32 && D != 64 && D != 128)
        return fail(DISM_ERR_UNSUPPORTED, "invalid vocabulary/channel size");
    if (vocab_head_stride != 0 && vocab_head_stride < V * D)
        return fail(DISM_ERR_INVALID, "%s: invalid vocabulary head stride", what);
    if ((reinterpret_cast<uintptr_t>(x) & 7) || (reinterpret_cast<uintptr_t>(vocab) & 15))
        return fail(DISM_ERR_INVALID, "%s: x must be 8-byte and vocab 16-byte aligned", what);
    return hip_status(dism::launch_vocab_argmax(x, vocab, vocab_head_stride, (int)B, (int)N,
                                                (int)H, (int)V, D, labels, scratch,
                                                S(stream)),
                      what);
}

}  // extern "C"

extern "C" {

int64_t dism_decoder_prime_workspace_bytes(int64_t B, int64_t n, int64_t H, int32_t R,
                                           int32_t DV, int32_t dtype) {
    const int64_t npad = (n + 255) / 256 * 256;
    if (n <= 0 || !dims_ok(B, npad, H) || B * H * npad > INT_MAX || !rdv_ok(R, DV) ||
        !dtype_ok(dtype))
        return -1;
    return layout(B, npad, H, R, DV).total + 2 * align256(B * H * npad * 4);
}

int32_t dism_decoder_prime(void* state, int64_t state_bytes, int64_t B, int64_t H, int32_t R,
                           int32_t DV, int64_t capacity, int32_t slots, int32_t dtype, int64_t n,
                           const int32_t* iq, const int32_t* ik, const uint8_t* reset,
                           const void* sk, const void* v, void* workspace,
                           int64_t workspace_bytes, void* stream) {
    const char* what = "decoder prime";
    if (int32_t lg = layout_guard()) return lg;
    if (!state || !iq || !ik || !sk || !v || !workspace)
        return fail(DISM_ERR_INVALID, "%s: null pointer", what);
    const int64_t rows = B * H;
    if (B <= 0 || H <= 0 || !decoder_dims_ok(rows, R, DV, capacity, slots, dtype))
        return fail(DISM_ERR_INVALID, "%s: invalid decoder dimensions", what);
    if (n <= 0 || n > capacity) return fail(DISM_ERR_INVALID, "%s: invalid token count", what);
    const int64_t need = dism_decoder_prime_workspace_bytes(B, n, H, R, DV, dtype);
    if (need < 0 || workspace_bytes < need)
        return fail(DISM_ERR_INVALID, "%s: workspace too small", what);
    if (!aligned16(sk) || !aligned16(v))
        return fail(DISM_ERR_INVALID, "%s: vectors must be 16-byte aligned", what);
    const DecoderLayout D = decoder_layout(rows, R, DV, capacity, slots, dtype);
    if (state_bytes < D.total) return fail(DISM_ERR_INVALID, "%s: state too small", what);
    const int64_t npad = (n + 255) / 256 * 256;
    const Layout L = layout(B, npad, H, R, DV);
    int32_t* pq = at<int32_t>(workspace, L.total);
    int32_t* pk = at<int32_t>(workspace, L.total + align256(rows * npad * 4));
    hipStream_t s = S(stream);
    int32_t st;
    if ((st = hip_status(dism::launch_pad_labels(iq, rows, n, npad, pq, s), what)) ||
        (st = hip_status(dism::launch_pad_labels(ik, rows, n, npad, pk, s), what)))
        return st;
    // combined label order of the padded prompt (the vectors are validated, not read)
    if ((st = dism_hard_prepare(sk, sk, v, dtype, pq, pk, B, npad, H, R, DV, workspace,
                                workspace_bytes, stream)))
        return st;
    dism::DecodeArgs a = decode_args(state, D, rows, H, R, DV, capacity, slots);
    a.n = (int)n;
    a.iq = iq;
    a.ik = ik;
    a.reset = reset;
    a.sk = sk;
    a.v = v;
    return hip_status(dism::launch_prime(a, orders(L, workspace), (int)npad, dtype, s), what);
}

}  // extern "C"
