// Fiber scheduler of the HIP CPU emulation (test infrastructure, see hip/hip_runtime.h).
#include "hip/hip_runtime.h"
#include <vector>
#include <algorithm>
#include <cassert>

extern "C" void emu_ctx_switch(void** from_sp, void* to_sp);
asm(R"(
.text
.globl emu_ctx_switch
.type emu_ctx_switch,@function
emu_ctx_switch:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
)");

namespace emu {
dim3 g_block_idx, g_grid_dim, g_block_dim;
hipError_t g_last_error = 0;

enum State { READY, BLOCKED, DONE };
enum Kind { K_BB = 0, K_WAVE = 1, K_SYNC = 2 };
constexpr int MAXDEPTH = 48;
struct Lane {
    dim3 tid;
    int id, lane, wave;
    State st;
    void* sp;
    unsigned char* stack;
    size_t stack_size;
    int op, arg, kind;
    uint64_t val, res;
    int depth;
    uintptr_t sig[MAXDEPTH];
    long nops;
};

Lane* g_cur = nullptr;
void* g_sched_sp = nullptr;
static std::vector<Lane> g_lanes;
static void (*g_body)(void*) = nullptr;
static void* g_ctx = nullptr;
static size_t g_stack_size = size_t(1) << 20;
static std::vector<unsigned char*> g_stacks;

Lane* cur() { return g_cur; }
static MfmaStage g_mfma[64];
MfmaStage& mfma_stage(int wave) { return g_mfma[wave & 63]; }
int wave_of_cur() { return g_cur->wave; }
const dim3& tid_of(Lane* l) { return l->tid; }
int lane_of_cur() { return g_cur->lane; }

static void lane_entry() {
    g_body(g_ctx);
    g_cur->st = DONE;
    emu_ctx_switch(&g_cur->sp, g_sched_sp);
    abort();
}

__attribute__((noinline)) void capture_sig(Lane* l, uintptr_t pc, uintptr_t* fp) {
    const uintptr_t lo = (uintptr_t)l->stack, hi = lo + l->stack_size;
    int d = 0;
    l->sig[d++] = pc;
    while (fp && (uintptr_t)fp >= lo && (uintptr_t)fp < hi && d < MAXDEPTH) {
        l->sig[d++] = fp[1];
        fp = (uintptr_t*)fp[0];
    }
    l->depth = d;
}

uint64_t wave_op(int kind, uint64_t value, int arg) {
    Lane* l = g_cur;
    l->op = kind;
    l->val = value;
    l->arg = arg;
    uintptr_t* fp = (uintptr_t*)__builtin_frame_address(0);
    capture_sig(l, fp[1], (uintptr_t*)fp[0]);
    l->kind = kind == OP_SYNC ? K_SYNC : K_WAVE;
    l->st = BLOCKED;
    emu_ctx_switch(&l->sp, g_sched_sp);
    return l->res;
}

// outermost frame first: lower return address = earlier code
static int cmp_sig(const Lane& a, const Lane& b) {
    int i = a.depth - 1, j = b.depth - 1;
    while (i >= 0 && j >= 0) {
        if (a.sig[i] != b.sig[j]) return a.sig[i] < b.sig[j] ? -1 : 1;
        --i; --j;
    }
    if (i < 0 && j < 0) return 0;
    return i < 0 ? -1 : 1;
}

static int dpp_src(int lane, int ctrl) {
    const int r = lane & ~15, i = lane & 15;
    if (ctrl <= 0xFF) {  // quad_perm
        const int q = lane & 3, base = lane & ~3;
        return base + ((ctrl >> (2 * q)) & 3);
    }
    if (ctrl == 0x141) return r + ((i & 8) | (7 - (i & 7)));  // row_half_mirror
    if (ctrl == 0x140) return r + (15 - i);                   // row_mirror
    if (ctrl >= 0x121 && ctrl <= 0x12F) return r + ((i + (ctrl - 0x120)) & 15);  // row_ror:n
    fprintf(stderr, "emu: unsupported dpp ctrl 0x%x\n", ctrl);
    abort();
}

static void resolve(std::vector<Lane*>& grp) {
    const int kind = grp[0]->op;
    uint64_t v[64] = {0};
    bool act[64] = {false};
    for (Lane* l : grp) {
        if (l->op != kind) {
            fprintf(stderr, "emu: lanes of one call site run different wave ops (%d/%d)\n", kind, l->op);
            abort();
        }
        v[l->lane] = l->val;
        act[l->lane] = true;
    }
    uint64_t ballot = 0;
    int first = 64;
    for (int i = 63; i >= 0; --i)
        if (act[i]) first = i;
    if (kind == OP_BALLOT)
        for (int i = 0; i < 64; ++i)
            if (act[i] && v[i]) ballot |= 1ull << i;
    for (Lane* l : grp) {
        const int i = l->lane, a = l->arg;
        uint64_t r = 0;
        auto get = [&](int s) -> uint64_t { return (s >= 0 && s < 64 && act[s]) ? v[s] : 0; };
        switch (kind) {
            case OP_BALLOT: r = ballot; break;
            case OP_SHFL: r = get(((a % 64) + 64) % 64); break;
            case OP_XOR: r = get(i ^ a); break;
            case OP_UP: {
                const int d = a & 255, w = a >> 8, seg = i - (i % w);
                r = (i - d >= seg) ? get(i - d) : v[i];
                break;
            }
            case OP_DOWN: {
                const int d = a & 255, w = a >> 8, seg = i - (i % w);
                r = (i + d < seg + w) ? get(i + d) : v[i];
                break;
            }
            case OP_FIRST: r = get(first); break;
            case OP_READLANE: r = get(a); break;
            case OP_BARRIER: case OP_SYNC: r = 0; break;
            case OP_DPP: r = (uint32_t)get(dpp_src(i, a)); break;
            case OP_PL16A: case OP_PL16B: {
                // rows of 16: vdst' = [a r0, b r0, a r2, b r2], vsrc' = [a r1, b r1, a r3, b r3]
                const int row = i >> 4, k = i & 15;
                const bool A = kind == OP_PL16A;
                int srow; bool useb;
                if (A) { srow = (row & 2) | 0; useb = row & 1; }
                else { srow = (row & 2) | 1; useb = row & 1; }
                const uint64_t w = get(srow * 16 + k);
                r = useb ? (w >> 32) : (w & 0xFFFFFFFFu);
                break;
            }
            case OP_PL32A: case OP_PL32B: {
                // vdst' = [a lo, b lo], vsrc' = [a hi, b hi]
                const int k = i & 31;
                const bool hiA = i >= 32;
                const int s = kind == OP_PL32A ? k : 32 + k;
                const uint64_t w = get(s);
                r = hiA ? (w >> 32) : (w & 0xFFFFFFFFu);
                break;
            }
            default: abort();
        }
        l->res = r;
        l->nops++;
    }
}

static void resume(Lane& l) {
    g_cur = &l;
    l.st = READY;
    emu_ctx_switch(&g_sched_sp, l.sp);
    g_cur = nullptr;
}

static void run_block() {
    const int n = (int)g_lanes.size();
    const int waves = (n + 63) / 64;
    for (int t = 0; t < n; ++t) resume(g_lanes[t]);  // every lane to its first stop
    std::vector<Lane*> cand, grp;
    for (;;) {
        bool progressed = false, live = false;
        for (int w = 0; w < waves; ++w) {
            cand.clear();
            for (int t = w * 64; t < n && t < w * 64 + 64; ++t) {
                Lane& l = g_lanes[t];
                if (l.st == DONE) continue;
                live = true;
                if (l.kind != K_SYNC) cand.push_back(&l);
            }
            if (cand.empty()) continue;
            Lane* best = cand[0];
            for (Lane* l : cand)
                if (cmp_sig(*l, *best) < 0) best = l;
            grp.clear();
            for (Lane* l : cand)
                if (cmp_sig(*l, *best) == 0) grp.push_back(l);
            if (best->kind == K_WAVE) resolve(grp);
            for (Lane* l : grp) resume(*l);
            progressed = true;
        }
        if (!live) return;
        if (progressed) continue;
        // only barriers left: release every live lane (with the predicate reductions)
        uint64_t any = 0, all = 1, cnt = 0;
        for (int t = 0; t < n; ++t)
            if (g_lanes[t].st != DONE) {
                any |= g_lanes[t].val;
                all &= g_lanes[t].val;
                cnt += g_lanes[t].val;
            }
        for (int t = 0; t < n; ++t)
            if (g_lanes[t].st != DONE) {
                Lane& l = g_lanes[t];
                l.res = l.arg == 1 ? any : l.arg == 2 ? all : l.arg == 3 ? cnt : 0;
                l.kind = K_BB;
            }
        for (int t = 0; t < n; ++t)
            if (g_lanes[t].st != DONE) resume(g_lanes[t]);
    }
}

void run_grid(void (*body)(void*), void* ctx, dim3 grid, dim3 block) {
    const int n = (int)(block.x * block.y * block.z);
    g_body = body;
    g_ctx = ctx;
    g_grid_dim = grid;
    g_block_dim = block;
    while ((int)g_stacks.size() < n) g_stacks.push_back((unsigned char*)malloc(g_stack_size));
    g_lanes.assign(n, Lane{});
    for (unsigned bz = 0; bz < grid.z; ++bz)
        for (unsigned by = 0; by < grid.y; ++by)
            for (unsigned bx = 0; bx < grid.x; ++bx) {
                g_block_idx = dim3(bx, by, bz);
                for (int t = 0; t < n; ++t) {
                    Lane& l = g_lanes[t];
                    l = Lane{};
                    l.id = t;
                    l.tid = dim3(t % block.x, (t / block.x) % block.y, t / (block.x * block.y));
                    l.lane = t & 63;
                    l.wave = t >> 6;
                    l.st = READY;
                    l.kind = K_BB;
                    l.stack = g_stacks[t];
                    l.stack_size = g_stack_size;
                    uintptr_t top = ((uintptr_t)(l.stack + g_stack_size)) & ~(uintptr_t)15;
                    void** sp = (void**)top;
                    *--sp = nullptr;
                    *--sp = (void*)&lane_entry;
                    for (int r = 0; r < 6; ++r) *--sp = nullptr;
                    l.sp = sp;
                }
                run_block();
            }
}
}  // namespace emu

#define EMU_ATOMIC_DEFS(T)                                                        \
    T atomicAdd(T* p, T v) { T o = *p; *p = o + v; return o; }                      \
    T atomicOr(T* p, T v) { T o = *p; *p = o | v; return o; }                       \
    T atomicMax(T* p, T v) { T o = *p; if (v > o) *p = v; return o; }               \
    T atomicMin(T* p, T v) { T o = *p; if (v < o) *p = v; return o; }               \
    T atomicExch(T* p, T v) { T o = *p; *p = v; return o; }                         \
    T atomicCAS(T* p, T c, T v) { T o = *p; if (o == c) *p = v; return o; }
EMU_ATOMIC_DEFS(int)
EMU_ATOMIC_DEFS(unsigned)
EMU_ATOMIC_DEFS(unsigned long long)
EMU_ATOMIC_DEFS(long long)
float atomicAdd(float* p, float v) { float o = *p; *p = o + v; return o; }
float atomicMax(float* p, float v) { float o = *p; if (v > o) *p = v; return o; }
float atomicExch(float* p, float v) { float o = *p; *p = v; return o; }

// basic-block hook (-fsanitize-coverage=trace-pc on the kernel units): every lane stops at
// every basic block; the scheduler runs a wave's lanes at the lowest code position one block
// at a time -- lockstep with reconvergence for structured control flow
extern "C" void __sanitizer_cov_trace_pc() {
    emu::Lane* l = emu::g_cur;
    if (!l) return;
    uintptr_t* fp = (uintptr_t*)__builtin_frame_address(0);
    emu::capture_sig(l, fp[1], (uintptr_t*)fp[0]);
    l->kind = emu::K_BB;
    l->st = emu::BLOCKED;
    emu_ctx_switch(&l->sp, emu::g_sched_sp);
}
