// Cooperative fiber runtime behind tests/emu/emu_hip.h (TEST INFRASTRUCTURE ONLY).
//
// A launch runs its workgroups one after another. A workgroup's threads are fibers on their own
// stacks, switched by a small x86-64 context switch; a fiber runs until it reaches a barrier or a
// cross-lane operation, where it waits for the other participants (the live threads of its
// workgroup or wavefront). The last one to arrive evaluates the operation for all of them. A
// wavefront whose lanes reach different cross-lane operations, or a barrier that some threads
// never reach, is reported as an error (it is undefined on the GPU).
//
// Global->LDS loads are asynchronous, as on the GPU: each lane queues its copies in issue order
// and they land in the LDS only when the wavefront waits for them (s_waitcnt with a vmcnt bound,
// a wave rendezvous that lands all but the newest N of every lane's copies), when the thread
// reaches __syncthreads() (whose release fence drains the counters), or when it exits. A plain
// s_barrier does not land them. A kernel that reads a stage of its LDS ring before waiting for
// it therefore reads what the slot held before, and its results are wrong on the CPU as well.
//
// LDS, static (__shared__ declarations, turned into references into an arena by the build) and
// dynamic, is refilled with a garbage pattern at the start of every workgroup.
//
// With EMU_TSAN (the ThreadSanitizer build; the kernels instrumented, this file not), every
// wavefront is one ThreadSanitizer fiber (its lanes run in lockstep on the GPU, so they are one
// thread of program order here, in the emulator's execution order; one fiber per lane would also
// exceed the sanitizer's slot count at 256-thread workgroups, which makes it drop its history),
// created afresh for each workgroup with fresh stacks, and the only happens-before edges are
// those the GPU provides: the launch before each wavefront; a workgroup barrier (arrivals before
// departures, per barrier generation); every wavefront before the end of the launch as the host
// sees it. Accesses of two workgroups of one launch,
// or of two wavefronts between barriers, that touch the same bytes with one of them a write
// and not both atomic are then reported as data races.
#include <sys/mman.h>

#include <unordered_map>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "emu_hip.h"

extern "C" void emu_swap(void** save_sp, void* next_sp);
asm(R"(
    .text
    .globl emu_swap
    .type emu_swap,@function
emu_swap:
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
    .size emu_swap, .-emu_swap
)");

#ifdef EMU_TSAN
extern "C" {
void* __tsan_get_current_fiber(void);
void* __tsan_create_fiber(unsigned flags);
void __tsan_destroy_fiber(void* fiber);
void __tsan_switch_to_fiber(void* fiber, unsigned flags);
void __tsan_acquire(void* addr);
void __tsan_release(void* addr);
void __tsan_read_range(void* addr, unsigned long size);
void __tsan_write_range(void* addr, unsigned long size);
void AnnotateIgnoreWritesBegin(const char* file, int line);
void AnnotateIgnoreWritesEnd(const char* file, int line);
}
#define TSAN(...) __VA_ARGS__
#else
#define TSAN(...)
#endif

namespace emu {
namespace {

#ifdef EMU_TSAN
constexpr size_t kStack = 128 << 10;     // per fiber, remapped for every workgroup
#else
constexpr size_t kStack = 1 << 20;       // per fiber (reserved lazily by the kernel)
#endif
constexpr size_t kLds = 160 * 1024;      // dynamic LDS of one workgroup
constexpr size_t kArena = 4 << 20;       // static LDS declarations of every kernel
constexpr int kMaxIn = 12;               // 32-bit words of a lane's operand (MFMA: a, b, c)

enum Kind { NONE = 0, SHFL, BALLOT, READLANE, READFIRST, DPP, MFMA, WBAR, VMWAIT };

constexpr int kMaxVm = 63;               // the vmcnt counter's range (issue stalls beyond it)

struct AsyncCopy {
    const void* src;
    uintptr_t dst;
    int size;
};

struct Fiber {
    void* sp = nullptr;
    char* stack = nullptr;
    Index tidx{0, 0, 0};
    int tid = 0;
    bool done = false;
    bool runnable = true;
    uint32_t in[kMaxIn];
    uint32_t out[4];
    bool pred = false;
    bool pending = false;      // waiting in a wave operation
    bool at_barrier = false;   // waiting in a workgroup barrier
    AsyncCopy q[kMaxVm];       // global->LDS copies in flight, oldest first (ring)
    int q_head = 0, q_len = 0;
    int bar_gen = 0;           // barrier generation this thread waits in
};

// Lands the oldest copies of `f` until at most `keep` remain.
void land_copies(Fiber& f, int keep) {
    while (f.q_len > keep) {
        const AsyncCopy& c = f.q[f.q_head];
        TSAN(__tsan_read_range(const_cast<void*>(c.src), c.size);
             __tsan_write_range(reinterpret_cast<void*>(c.dst), c.size);)
        memcpy(reinterpret_cast<void*>(c.dst), c.src, c.size);
        f.q_head = (f.q_head + 1) % kMaxVm;
        f.q_len--;
    }
}

struct WaveOp {
    Kind kind = NONE;
    int p0 = 0, p1 = 0, p2 = 0, p3 = 0;
    int arrived = 0;
    uint64_t mask = 0;   // lanes waiting
};

struct State {
    std::function<void()>* body = nullptr;
    std::vector<Fiber> fibers;
    std::vector<WaveOp> waves;
    int nthreads = 0;
    int bar_arrived = 0;
    int bar_gen = 0;
    char* arena = nullptr;               // static LDS (below 4 GiB, like the dynamic LDS)
    size_t arena_used = 0;
    std::unordered_map<uint64_t, size_t> arena_at;   // (declaration, size) -> offset
    void* tsan_main = nullptr;
    char* tokens = nullptr;              // this workgroup's synchronisation addresses
    char* end_token = nullptr;           // the launch's: every thread -> the host
    std::vector<void*> wave_tsan;        // ThreadSanitizer fiber per wavefront (EMU_TSAN)
    Index bidx{0, 0, 0}, bdim{1, 1, 1}, gdim{1, 1, 1};
    Fiber* cur = nullptr;
    void* sched_sp = nullptr;
    char* lds = nullptr;
    hipError_t err = hipSuccess;
    std::string msg;
};

State S;

// Synchronisation addresses of the current workgroup (EMU_TSAN), fresh for each workgroup so
// that no edge leads from one workgroup to another: [0] launch, [2..3] barrier generations
// ([1] unused; the end of the launch has its own address).
void* token(int i) { return S.tokens + i; }

[[noreturn]] void fail(const std::string& m) {
    fprintf(stderr, "emu: %s (block %u,%u,%u thread %d)\n", m.c_str(), S.bidx.x, S.bidx.y,
            S.bidx.z, S.cur ? S.cur->tid : -1);
    fflush(stderr);
    abort();
}

char* map_low(size_t bytes) {
    void* p = mmap(nullptr, bytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_32BIT,
                   -1, 0);
    if (p == MAP_FAILED) fail("cannot map LDS below 4 GiB");
    return static_cast<char*>(p);
}

char* low_lds() {
    if (!S.lds) S.lds = map_low(kLds);
    return S.lds;
}

void try_complete_wave(int w);
void try_complete_barrier();
int wave_of(const Fiber* f) { return f->tid / 64; }

// Switches from the running thread to the scheduler.
void to_scheduler(Fiber* f) {
    TSAN(__tsan_switch_to_fiber(S.tsan_main, 1);)
    emu_swap(&f->sp, S.sched_sp);
}

void yield_blocked() {
    Fiber* f = S.cur;
    f->runnable = false;
    to_scheduler(f);
}

void fiber_entry() {
    TSAN(__tsan_acquire(token(0));)
    (*S.body)();
    Fiber* f = S.cur;
    land_copies(*f, 0);   // loads still in flight at the end of the program land regardless
    TSAN(__tsan_release(S.end_token);)
    f->done = true;
    // a finished thread no longer takes part in its workgroup's barrier or its wave's ops
    try_complete_wave(wave_of(f));
    try_complete_barrier();
    to_scheduler(f);
    fail("finished fiber resumed");
}

uint64_t live_lanes(int w) {
    uint64_t m = 0;
    for (int l = 0; l < 64; ++l) {
        const int t = w * 64 + l;
        if (t < S.nthreads && !S.fibers[t].done) m |= 1ull << l;
    }
    return m;
}

void complete_wave(int w);

void try_complete_wave(int w) {
    WaveOp& op = S.waves[w];
    if (op.kind == NONE) return;
    const uint64_t live = live_lanes(w);
    if ((op.mask & live) == live && op.mask != 0) complete_wave(w);
}

void try_complete_barrier() {
    int live = 0;
    for (int t = 0; t < S.nthreads; ++t) live += !S.fibers[t].done;
    if (S.bar_arrived > 0 && S.bar_arrived == live) {
        S.bar_arrived = 0;
        S.bar_gen++;
        for (int t = 0; t < S.nthreads; ++t)
            if (!S.fibers[t].done) {
                S.fibers[t].at_barrier = false;
                S.fibers[t].runnable = true;
            }
    }
}

uint32_t lane_in(int w, int l, int i) {
    const int t = w * 64 + l;
    if (t >= S.nthreads || S.fibers[t].done) return 0;   // an exited lane reads as zero
    return S.fibers[t].in[i];
}

int dpp_source(int l, int ctrl, bool& valid) {
    valid = true;
    if (ctrl <= 0xFF) return (l & ~3) | ((ctrl >> (2 * (l & 3))) & 3);   // quad_perm
    if (ctrl == 0x140) return (l & ~15) | (15 - (l & 15));                 // row_mirror
    if (ctrl == 0x141) return (l & ~7) | (7 - (l & 7));                    // row_half_mirror
    const int row = l >> 4;
    if (ctrl == 0x142) {                                                   // row_bcast:15
        if (row == 0) valid = false;
        return (row - 1) * 16 + 15;
    }
    if (ctrl == 0x143) {                                                   // row_bcast:31
        if (row < 2) valid = false;
        return 31;
    }
    fail("DPP control " + std::to_string(ctrl) + " not emulated");
}

void complete_wave(int w) {
    WaveOp& op = S.waves[w];
    const uint64_t mask = op.mask;
    for (int l = 0; l < 64; ++l) {
        if (!(mask >> l & 1)) continue;
        Fiber& f = S.fibers[w * 64 + l];
        switch (op.kind) {
            case SHFL: {
                const int width = op.p1, arg = (int)f.in[1];
                const int base = l & ~(width - 1);
                int src = l;
                if (op.p2 == 0) src = base + (((l - base) ^ arg) & (width - 1));
                else if (op.p2 == 1) src = base + (arg & (width - 1));
                else if (op.p2 == 2) src = (l - base) >= arg ? l - arg : l;
                else src = (l - base) + arg < width ? l + arg : l;
                f.out[0] = lane_in(w, src, 0);
                break;
            }
            case BALLOT: {
                uint64_t b = 0;
                for (int j = 0; j < 64; ++j) {
                    const int t = w * 64 + j;
                    if (t < S.nthreads && (mask >> j & 1) && S.fibers[t].pred) b |= 1ull << j;
                }
                f.out[0] = (uint32_t)b;
                f.out[1] = (uint32_t)(b >> 32);
                break;
            }
            case READLANE:
                f.out[0] = lane_in(w, op.p0 & 63, 0);
                break;
            case READFIRST: {
                int first = __builtin_ctzll(mask);
                f.out[0] = lane_in(w, first, 0);
                break;
            }
            case DPP: {
                const int row = l >> 4;
                if (!(op.p1 >> row & 1)) { f.out[0] = f.in[0]; break; }   // row masked: old
                bool valid;
                const int s = dpp_source(l, op.p0, valid);
                f.out[0] = valid ? lane_in(w, s, 1) : (op.p3 ? 0u : f.in[0]);
                break;
            }
            case VMWAIT:
                land_copies(f, op.p0);
                break;
            case MFMA:
            case WBAR:
                break;
            default:
                fail("bad wave op");
        }
    }
    if (op.kind == MFMA) {
        if (mask != ~0ull) fail("MFMA with inactive lanes");
        // A[m][k]: lane m % 16 + 16 * (k / 8), element k % 8; B[k][n] likewise (kept as
        // Bt[n][k]); D[m][n]: lane n + 16 * (m / 4), element m % 4. fp32 products and sums.
        alignas(32) float A[16][32], Bt[16][32];
        for (int l = 0; l < 64; ++l) {
            const Fiber& f = S.fibers[w * 64 + l];
            const uint16_t* a = reinterpret_cast<const uint16_t*>(&f.in[0]);
            const uint16_t* b = reinterpret_cast<const uint16_t*>(&f.in[4]);
            for (int i = 0; i < 8; ++i) {
                A[l % 16][8 * (l / 16) + i] = __builtin_bit_cast(float, (uint32_t)a[i] << 16);
                Bt[l % 16][8 * (l / 16) + i] = __builtin_bit_cast(float, (uint32_t)b[i] << 16);
            }
        }
        for (int l = 0; l < 64; ++l) {
            Fiber& f = S.fibers[w * 64 + l];
            const int n = l % 16;
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * (l / 16) + i;
                float acc = 0.0f;
                for (int k = 0; k < 32; ++k) acc += A[m][k] * Bt[n][k];
                f.out[i] = __builtin_bit_cast(uint32_t, acc + __builtin_bit_cast(float, f.in[8 + i]));
            }
        }
    }
    op = WaveOp{};
    for (int l = 0; l < 64; ++l)
        if (mask >> l & 1) {
            S.fibers[w * 64 + l].pending = false;
            S.fibers[w * 64 + l].runnable = true;
        }
}

// Arrive at a wave operation; returns after the operation completed.
void wave_arrive(Kind k, int p0 = 0, int p1 = 0, int p2 = 0, int p3 = 0) {
    Fiber* f = S.cur;
    const int w = wave_of(f), l = f->tid & 63;
    WaveOp& op = S.waves[w];
    if (op.kind == NONE) {
        op.kind = k;
        op.p0 = p0;
        op.p1 = p1;
        op.p2 = p2;
        op.p3 = p3;
    } else if (op.kind != k || op.p0 != p0 || op.p1 != p1 || op.p2 != p2 || op.p3 != p3) {
        fail("lanes of a wavefront reached different cross-lane operations");
    }
    op.mask |= 1ull << l;
    op.arrived++;
    f->pending = true;
    try_complete_wave(w);
    while (f->pending) yield_blocked();
}

}  // namespace

const Index& thread_idx() { return S.cur->tidx; }
const Index& block_idx() { return S.bidx; }
const Index& block_dim() { return S.bdim; }
const Index& grid_dim() { return S.gdim; }
int lane() { return S.cur->tid & 63; }
char* dynamic_lds() { return low_lds(); }

void* static_lds(int key, size_t bytes, size_t align) {
    const uint64_t k = (uint64_t)key << 40 | bytes;
    auto it = S.arena_at.find(k);
    if (it == S.arena_at.end()) {
        const size_t a = align < 16 ? 16 : align;
        const size_t off = (S.arena_used + a - 1) / a * a;
        if (off + bytes > kArena) fail("static LDS arena exhausted");
        S.arena_used = off + bytes;
        // the fill stands for the state the workgroup finds, not for an access of this thread
        TSAN(AnnotateIgnoreWritesBegin(__FILE__, __LINE__);)
        memset(S.arena + off, 0xFF, bytes);
        TSAN(AnnotateIgnoreWritesEnd(__FILE__, __LINE__);)
        it = S.arena_at.emplace(k, off).first;
    }
    return S.arena + it->second;
}
hipError_t last_error() {
    const hipError_t e = S.err;
    S.err = hipSuccess;
    return e;
}

void barrier_arrive() {
    Fiber* f = S.cur;
    f->bar_gen = S.bar_gen;
    TSAN(__tsan_release(token(2 + (f->bar_gen & 1)));)
    S.bar_arrived++;
    f->at_barrier = true;
    try_complete_barrier();
    while (f->at_barrier) yield_blocked();
    TSAN(__tsan_acquire(token(2 + (f->bar_gen & 1)));)
}

void syncthreads() {
    land_copies(*S.cur, 0);   // __syncthreads' release fence waits for the vector counters
    barrier_arrive();
}

void s_barrier() { barrier_arrive(); }

void s_waitcnt(int imm) {
    // gfx9 encoding: vmcnt in bits 3:0 and 15:14; only the vector-memory count is modelled
    // (LDS and scalar accesses complete at once here)
    const int vm = (imm & 15) | (((imm >> 14) & 3) << 4);
    if (vm >= kMaxVm) return;
    wave_arrive(VMWAIT, vm);
}

void wave_barrier() { wave_arrive(WBAR); }

uint32_t shfl_u32(uint32_t v, int arg, int mode, int width) {
    S.cur->in[0] = v;
    S.cur->in[1] = (uint32_t)arg;   // per lane: __shfl takes a lane-varying source
    wave_arrive(SHFL, mode == 1 ? 0 : arg, width, mode);
    return S.cur->out[0];
}

uint64_t ballot(bool p) {
    S.cur->pred = p;
    wave_arrive(BALLOT);
    return (uint64_t)S.cur->out[0] | ((uint64_t)S.cur->out[1] << 32);
}

uint32_t readlane_u32(uint32_t v, int l) {
    S.cur->in[0] = v;
    wave_arrive(READLANE, l);
    return S.cur->out[0];
}

uint32_t readfirstlane_u32(uint32_t v) {
    S.cur->in[0] = v;
    wave_arrive(READFIRST);
    return S.cur->out[0];
}

uint32_t update_dpp_u32(uint32_t old, uint32_t src, int ctrl, int row_mask, int bank_mask,
                        bool bound_ctrl) {
    if (bank_mask != 0xF) fail("DPP bank masks are not emulated");
    S.cur->in[0] = old;
    S.cur->in[1] = src;
    wave_arrive(DPP, ctrl, row_mask, 0, bound_ctrl);
    return S.cur->out[0];
}

void mfma_16x16x32_bf16(const void* a, const void* b, const float* c, float* d) {
    memcpy(&S.cur->in[0], a, 16);
    memcpy(&S.cur->in[4], b, 16);
    memcpy(&S.cur->in[8], c, 16);
    wave_arrive(MFMA);
    memcpy(d, S.cur->out, 16);
}

void global_load_lds(const void* g, uintptr_t lds, int size, int offset) {
    const uintptr_t lo = (uintptr_t)low_lds();
    const uintptr_t dst = lds + offset + (uintptr_t)lane() * size;
    if (dst < lo || dst + size > lo + kLds) fail("global_load_lds outside the LDS");
    Fiber& f = *S.cur;
    if (f.q_len == kMaxVm) land_copies(f, kMaxVm - 1);   // the counter is full: issue waits
    f.q[(f.q_head + f.q_len) % kMaxVm] = AsyncCopy{g, dst, size};
    f.q_len++;
}

void launch(dim3 grid, dim3 block, size_t dyn_lds, std::function<void()> body) {
    if (block.y != 1 || block.z != 1) fail("only 1-D workgroups are emulated");
    if (dyn_lds > kLds) {
        S.err = hipErrorInvalidValue;
        return;
    }
    const int n = (int)block.x;
    if (n < 1 || n > 1024) {
        S.err = hipErrorInvalidValue;
        return;
    }
    S.body = &body;
    S.nthreads = n;
    S.bdim = Index{block.x, 1, 1};
    S.gdim = Index{grid.x, grid.y, grid.z};
    S.fibers.assign(n, Fiber{});
    S.waves.assign((n + 63) / 64, WaveOp{});
    std::vector<char*> stacks(n);
    for (int t = 0; t < n; ++t) {
        stacks[t] = static_cast<char*>(mmap(nullptr, kStack, PROT_READ | PROT_WRITE,
                                            MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0));
        if (stacks[t] == MAP_FAILED) fail("cannot map a fiber stack");
    }
    low_lds();
    // mapped here, by the host side: a mapping is an access of the thread that makes it
    if (!S.arena) S.arena = map_low(kArena);
#ifdef EMU_TSAN
    S.tsan_main = __tsan_get_current_fiber();
    S.end_token = static_cast<char*>(malloc(1));
    if (!S.end_token) fail("out of memory");
#endif
    for (unsigned bz = 0; bz < grid.z; ++bz)
        for (unsigned by = 0; by < grid.y; ++by)
            for (unsigned bx = 0; bx < grid.x; ++bx) {
                S.bidx = Index{bx, by, bz};
#ifdef EMU_TSAN
                // this workgroup's memory is new to it: fresh stacks, LDS history forgotten
                for (int t = 0; t < n; ++t) {
                    munmap(stacks[t], kStack);
                    stacks[t] = static_cast<char*>(mmap(nullptr, kStack, PROT_READ | PROT_WRITE,
                                                        MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE,
                                                        -1, 0));
                    if (stacks[t] == MAP_FAILED) fail("cannot map a fiber stack");
                }
                munmap(S.lds, kLds);   // the interceptors forget the old mappings' history
                S.lds = map_low(kLds);
                munmap(S.arena, kArena);
                S.arena = map_low(kArena);
                S.tokens = static_cast<char*>(malloc(4));
                if (!S.tokens) fail("out of memory");
                S.wave_tsan.assign(S.waves.size(), nullptr);
                for (auto& wf : S.wave_tsan) wf = __tsan_create_fiber(0);
#endif
                memset(S.lds, 0xFF, kLds);   // LDS starts as garbage (NaN patterns)
                memset(S.arena, 0xFF, S.arena_used);
                S.bar_gen = 0;
                S.bar_arrived = 0;
                for (auto& w : S.waves) w = WaveOp{};
                for (int t = 0; t < n; ++t) {
                    Fiber& f = S.fibers[t];
                    f = Fiber{};
                    f.tid = t;
                    f.tidx = Index{(unsigned)t, 0, 0};
                    uintptr_t top = ((uintptr_t)stacks[t] + kStack) & ~(uintptr_t)15;
                    uint64_t* sp = reinterpret_cast<uint64_t*>(top);
                    *--sp = 0;                                    // fake return address
                    *--sp = (uint64_t)(uintptr_t)&fiber_entry;    // emu_swap's ret target
                    for (int r = 0; r < 6; ++r) *--sp = 0;        // rbp rbx r12-r15
                    f.sp = sp;
                }
                TSAN(__tsan_release(token(0));)
                for (;;) {
                    bool progress = false, all_done = true;
                    for (int t = 0; t < n; ++t) {
                        Fiber& f = S.fibers[t];
                        if (f.done) continue;
                        all_done = false;
                        if (!f.runnable) continue;
                        S.cur = &f;
                        TSAN(__tsan_switch_to_fiber(S.wave_tsan[t / 64], 1);)
                        emu_swap(&S.sched_sp, f.sp);
                        S.cur = nullptr;
                        progress = true;
                    }
                    if (all_done) break;
                    if (!progress) fail("deadlock: a barrier or wave operation never completes");
                }
#ifdef EMU_TSAN
                for (void* wf : S.wave_tsan) __tsan_destroy_fiber(wf);
                free(S.tokens);             // drops this workgroup's synchronisation state
                S.tokens = nullptr;
#endif
            }
    for (int t = 0; t < n; ++t) munmap(stacks[t], kStack);
#ifdef EMU_TSAN
    __tsan_acquire(S.end_token);   // the host sees the whole launch complete
    free(S.end_token);
    S.end_token = nullptr;
#endif
    S.body = nullptr;
}

}  // namespace emu
