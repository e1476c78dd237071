// LDS-pipelined grouped GEMMs for prefill-sized batches (64/128/256-row expert tiles).
//
// Workgroup tile: BM expert-sorted rows x 256 rows of B (gate_up: 8 gate + 8 up 16-row blocks ->
// 128 activation columns; down: 256 output columns), 8 wavefronts in a WM x (8/WM) grid (WM = 1
// for 64 rows, 2 for 128 and 256), each owning a (BM/WM) x (256*WM/8) block of C in 16x16x32
// bf16 MFMA accumulators. A 256-row tile reads each weight panel once for both 128-row halves
// of an expert's rows (a half of padding rows only is skipped), at the cost of streaming its A
// fragments in halves to fit the accumulators in the register budget.
//
// Operands reach LDS through direct global->LDS loads (global_load_lds_dwordx4: 64 lanes x 16 B,
// written to LDS at lane*16), in stages of 64 k through a ring of NS stages:
//   - B comes from the MFMA-tiled (packed) weights, where a 16-row x 32-k operand block is 1 KiB
//     of contiguous memory already in MFMA lane order;
//   - A rows (gate_up: gathered x[sorted_id / top_k]; down: activation rows) are loaded as whole
//     128-byte lines, 8 rows per instruction: through the texture path a gather of whole lines
//     runs about three times faster than one of half lines (16 rows x 64 B per instruction). The
//     16-byte chunks are XOR-swizzled across lanes so that the 16 lanes of an MFMA operand read
//     hit 16 distinct LDS bank groups: lane' = rr*8 + (c ^ ((rr >> 1) | (h << 2))) holds row rr
//     (0..7) of the instruction's 8-row group, 16-byte chunk c, where h is the group's half of
//     its 16-row block.
// The grid is persistent (one workgroup per CU, the ring fills the LDS): each workgroup walks a
// strided list of tiles within its XCD's contiguous share of the tile space, and issues the first
// stages of its next tile before running the epilogue of the current one, so the pipeline's
// fill latency hides behind the epilogue stores.
// Reference computation: _fused_moe_kernel (tinykernels.py:1589-1765), epilogues as in the
// weight-streaming kernels (SwiGLU with the reference's bf16 rounding points; routing-weight
// scaling and scatter to assignment order).
#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt in bits 3:0
// and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima). vmcnt also counts stores; loads
// retire in issue order, so "at most N outstanding" implies that every load but the last N
// issued has landed.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The compiler does not order LDS reads after the global->LDS loads that fill them, and
// __syncthreads() would drain every outstanding load (a release fence) before each barrier. The
// ring is therefore synchronised by hand: each wavefront waits (vmcnt) for its own loads of the
// stage it is about to read and for its own LDS reads of the previous stage (lgkmcnt), then a
// plain s_barrier publishes the stage to every wavefront and frees the slot the next loads
// overwrite. The asm statements carry "memory" clobbers so no LDS access moves across them.
__device__ __forceinline__ u32x4 lds_read16(uint32_t addr) {
    return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(addr);
}
__device__ __forceinline__ void lds_write2(uint32_t addr, bf16_t v) {
    *reinterpret_cast<__attribute__((address_space(3))) bf16_t*>(addr) = v;
}
// Copies a loaded value into a fresh register: the compiler places its wait for the load here,
// where nothing else is in flight, instead of at a later use behind the next tile's loads.
__device__ __forceinline__ int settle(int v) {
    int r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}
__device__ __forceinline__ float settle(float v) {
    float r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}
__device__ __forceinline__ void barrier_after_lds_reads() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int kBN = 256;     // B rows per tile
constexpr int kBlk = 1024;   // bytes per load instruction (and per 16x32 operand block)
constexpr int kNW = 8;       // wavefronts per workgroup

// swizzle of the 16-byte chunks of row rr in half h of a 16-row block
__device__ __forceinline__ int a_swz(int rr, int h) { return (rr >> 1) | (h << 2); }

// Interleave the next k-step's LDS reads (NR) with this k-step's MFMAs (NM) in the instruction
// stream, so that each wavefront keeps the matrix core busy while its operand reads are in
// flight (wavefronts reach the stage barrier together, so overlap across wavefronts alone leaves
// the LDS-bound and MFMA-bound phases of a stage serialised).
template <int NR, int NM>
__device__ __forceinline__ void interleave_reads_mfma() {
    // One MFMA leads each read, and the region ends with MFMAs only: the conservative
    // lgkmcnt(0) the compiler places before a region's first MFMA then finds the previous
    // region's reads long landed instead of waiting on a read issued just before it.
    static_assert(NM > NR, "more MFMAs than reads per k-step");
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NM - NR, 0);
}

// Schedule of a 256-row tile's second half-k-step: the FH reads of the next A half interleaved
// with the first FH MFMAs (B block 0), then after each B block's FH MFMAs the read that refills
// that block's B fragment for the next k-step (its last use has then issued).
template <int FH, int FN>
__device__ __forceinline__ void refill_sched() {
#pragma unroll
    for (int i = 0; i < FH; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
    for (int g = 1; g < FN; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x008, FH, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
}

// Ring: A (gathered rows) in 2 slots, B (weights, the operand streamed from HBM) in NB slots, so
// B runs NB - 1 stages ahead and A one stage ahead. Issue order per tile: B(0..NB-3), A(0),
// B(NB-2), then at the barrier before stage s (s >= 1) A(s+1), B(s+NB-1). When the wavefront
// waits for stage s, the only loads it has issued after A(s) are those of B(s+NB-2), if any.
template <int BM, bool GATEUP, int WM, int NB>
__global__ __launch_bounds__(64 * kNW, 1) void moe_tile_kernel(GemmArgs p) {
    constexpr int NT = 64 * kNW;
    constexpr int WN = kNW / WM;            // wavefront columns (WM wavefront rows)
    constexpr int FM = BM / 16 / WM;        // A row blocks per wavefront
    constexpr int NBK = kBN / 16;           // B row blocks per tile (16)
    constexpr int FN = NBK / WN;            // B blocks per wavefront
    constexpr int A_INST = BM / 8;          // A load instructions per stage (8 rows x 128 B)
    constexpr int LPA = A_INST / kNW;       // A loads per wavefront per stage
    constexpr int LPB = 2 * NBK / kNW;      // B loads per wavefront per stage (4)
    constexpr int A_BYTES = A_INST * kBlk;
    constexpr int B_BYTES = 2 * NBK * kBlk;
    constexpr int LB = NB - 1;              // B lookahead in stages
    constexpr int NR = FM + FN;             // LDS reads per k-step
    constexpr int NM = FM * FN;             // MFMAs per k-step
    static_assert(A_INST % kNW == 0 && LPA >= 1, "A loads must split evenly over the wavefronts");
    static_assert(LB >= 2, "B must run at least two stages ahead (wait accounting)");
    static_assert(!GATEUP || FN % 2 == 0, "gate/up block pairs per wavefront");
    static_assert(FM * 16 * WM == BM && FN * WN == NBK, "wavefront grid must cover the tile");
    static_assert(2 * A_BYTES + NB * B_BYTES <= 160 * 1024, "LDS budget");
    // Epilogue staging: C rows go through B slot NB-1 (the next tile's prologue fills only
    // slots 0..NB-2), RP rows per pass, then leave as 16-byte row chunks.
    constexpr int OUTC_C = GATEUP ? kBN / 2 : kBN;   // C columns per tile
    constexpr int ROWB = OUTC_C * 2;                 // bytes per staged row
    constexpr int RP = B_BYTES / ROWB < BM ? B_BYTES / ROWB : BM;
    constexpr int NPASS = BM / RP;
    constexpr int CPR = ROWB / 16;                   // 16-byte chunks per row
    constexpr int CPL = RP * CPR / NT;               // chunks per lane per pass
    static_assert(RP * CPR % NT == 0 && BM % RP == 0, "epilogue passes");
    extern __shared__ __attribute__((aligned(1024))) char lds[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int KS = p.K / 32;                // k-steps
    const int NST = p.K / 64;               // stages
    const int OUTC = GATEUP ? kBN / 2 : kBN;

    // Tiles that hold rows: the align step fills total[0] padded rows.
    const int valid_m = min((p.total[0] + BM - 1) / BM, p.m_tiles);
    const int G = valid_m * p.n_tiles;
    const int xcd = blockIdx.x & 7, per_xcd = gridDim.x >> 3, slot = blockIdx.x >> 3;
    const int q8 = G >> 3, r8 = G & 7;
    const int chunk_begin = xcd * q8 + min(xcd, r8);
    const int chunk_end = chunk_begin + q8 + (xcd < r8 ? 1 : 0);

    // Load sources. A: wavefront w issues the 8-row groups w + 8j (element offsets of each lane's
    // row and swizzled chunk; gate_up rows are gathered from all of x, so 64-bit, while down's
    // rows are the tile's own consecutive rows, so a 32-bit offset from the tile's first row,
    // a_base, which is uniform). B: instruction index w + 8j is block (nb, kk) = ((w >> 1) + 4j,
    // w & 1), so one base pointer plus j * b_jstride covers the wavefront's loads.
    // 256-row gate_up tiles use 32-bit offsets too (x below 4 GiB, checked on the host): the
    // loads then take the uniform base in SGPRs and one offset VGPR (the register budget of
    // these tiles has no room for 64-bit addresses).
    using a_off_t = typename std::conditional<GATEUP && BM != 256, uint64_t, uint32_t>::type;
    a_off_t a_src[LPA];
    const bf16_t* a_base = p.A;
    const bf16_t* b_src = nullptr;
    int64_t b_jstride = 0;
    int expert = -1, m0 = 0, n_tile = 0;
    // down: assignment of tile row `tid` (tid < BM), loaded with the tile's other setup reads
    int row_flat = 0;
    // Tile setup in two halves: fetch() issues the reads a tile's loads depend on (its expert,
    // and the assignment of the rows this lane gathers (gate_up) or of row `tid` (down)); for
    // the next tile they are issued at the top of the current one, so their latency hides behind
    // its stages, and settled after its last stage, when nothing else is in flight. finish()
    // turns them into load sources.
    int f_m0 = 0, f_n = 0, f_expert = -1, f_rowflat = 0;
    // gate_up: the sorted ids of the rows this lane gathers (load j: row (wave + 8 j) * 8 +
    // lane / 8). 256-row tiles, whose registers are the scarcest, hold one id per lane instead
    // (lane l: load l / 8 % 4, row l % 8) and move them to their loaders with a shuffle.
    constexpr int NFL = BM == 256 ? 1 : LPA;
    int f_flat[NFL];
    auto fetch = [&](int logical) {
        // column tiles fastest: the tiles that share an A block run side by side, and so do
        // the row tiles of one expert that share a B panel
        const int m_tile = logical / p.n_tiles;
        f_n = logical % p.n_tiles;
        f_m0 = m_tile * BM;
        f_expert = p.expert_ids[m_tile];
        if (GATEUP) {
#pragma unroll
            for (int j = 0; j < LPA; ++j)
                if (BM == 256) {
                    if (j == 0)
                        f_flat[0] = p.sorted_ids[f_m0 + (wave + ((lane >> 3) & 3) * kNW) * 8 +
                                                 (lane & 7)];
                } else {
                    f_flat[j] = p.sorted_ids[f_m0 + (wave + j * kNW) * 8 + (lane >> 3)];
                }
        } else {
            f_rowflat = tid < BM ? p.sorted_ids[f_m0 + tid] : (int)p.numel;
        }
    };
    auto settle_fetch = [&]() {
        f_expert = settle(f_expert);
        if (GATEUP) {
#pragma unroll
            for (int j = 0; j < NFL; ++j) f_flat[j] = settle(f_flat[j]);
        } else {
            f_rowflat = settle(f_rowflat);
        }
    };
    auto finish = [&]() {
        m0 = f_m0;
        n_tile = f_n;
        expert = __builtin_amdgcn_readfirstlane(f_expert);
        row_flat = f_rowflat;
        if (expert < 0) return;
        const int rr = lane >> 3;
        const int c = (lane & 7) ^ a_swz(rr, wave & 1);
#pragma unroll
        for (int j = 0; j < LPA; ++j) {
            int src_row;
            if (GATEUP) {
                int flat = BM == 256 ? __shfl(f_flat[0], j * 8 + (lane >> 3)) : f_flat[j];
                if (flat >= p.numel) flat = 0;  // padding row: any valid row, discarded
                src_row = flat / p.top_k;
            } else {
                src_row = (wave + j * kNW) * 8 + rr;
            }
            a_src[j] = (a_off_t)src_row * (a_off_t)p.K + c * 8;
        }
        if (!GATEUP) a_base = p.A + (int64_t)m0 * p.K;
        const bf16_t* Be = p.B + (int64_t)expert * (GATEUP ? 2 : 1) * p.N * p.K;
        b_src = Be + ((int64_t)(n_tile * NBK + (wave >> 1)) * KS + (wave & 1)) * 512 + lane * 8;
        b_jstride = (int64_t)4 * KS * 512;
    };
    auto issue_a = [&](int st) {
        char* base = lds + (st & 1) * A_BYTES;
        // 256: the base is made opaque to the loop so the compiler cannot hoist 64-bit
        // addresses (two registers each) out of it; base + 32-bit byte offset selects the
        // load form with the base in SGPRs
        const bf16_t* ab = a_base;
        if constexpr (BM == 256) asm volatile("" : "+s"(ab));
#pragma unroll
        for (int j = 0; j < LPA; ++j)
            __builtin_amdgcn_global_load_lds(
                BM == 256 ? (const void*)((const char*)ab + (uint32_t)(a_src[j] * 2u + st * 128u))
                          : (const void*)(a_base + a_src[j] + st * 64),
                (lds_void*)(base + (wave + j * kNW) * kBlk), 16, 0, 0);
    };
    auto issue_b = [&](int st) {
        char* base = lds + 2 * A_BYTES + (st % NB) * B_BYTES;
#pragma unroll
        for (int j = 0; j < LPB; ++j)
            __builtin_amdgcn_global_load_lds(
                (const void*)(b_src + j * b_jstride + (int64_t)st * 1024),
                (lds_void*)(base + (wave + j * kNW) * kBlk), 16, 0, 0);
    };
    auto prologue = [&]() {
#pragma unroll
        for (int s = 0; s + 1 < LB; ++s)
            if (s < NST) issue_b(s);
        issue_a(0);
        if (LB - 1 < NST) issue_b(LB - 1);
    };

    // LDS byte offsets this lane reads: A block (mb, kk) at mb*2048 + a_off[kk] within an A slot;
    // B block (nb, kk) at (nb*2 + kk) * 1024 + lane*16 within a B slot.
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)lds;
    uint32_t a_off[2];
    {
        const int r = lane & 15, q = lane >> 4, h = r >> 3, rr = r & 7;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
            a_off[kk] = h * kBlk + (rr * 8 + ((kk * 4 + q) ^ a_swz(rr, h))) * 16;
    }
    auto read_frags = [&](int st, int kk, u32x4 (&af)[FM], u32x4 (&bfr)[FN]) {
        const uint32_t ab = lds0 + (st & 1) * A_BYTES + a_off[kk];
        const uint32_t bb = lds0 + 2 * A_BYTES + (st % NB) * B_BYTES + kk * kBlk + lane * 16;
#pragma unroll
        for (int f = 0; f < FM; ++f) af[f] = lds_read16(ab + (wm * FM + f) * 2 * kBlk);
#pragma unroll
        for (int g = 0; g < FN; ++g) bfr[g] = lds_read16(bb + (wn * FN + g) * 2 * kBlk);
    };

    // Tile order: each expert's tiles column-major, i.e. the row tiles that share a weight panel
    // are adjacent in the list, so the tiles an XCD runs at once span few panels and few panels
    // straddle two consecutive rounds (row-major order re-fetched about one expert's panels per
    // round). The workgroup remaps its strided tile list once, at start: expert_ids goes into
    // LDS (before the ring uses it), each lane k binary-searches the bucket of its k-th tile
    // (expert_ids is non-decreasing with the remote bucket's -1 taken as +inf) and keeps the
    // plain index (row tile * n_tiles + column tile). Lists longer than 128 tiles per workgroup,
    // or tables larger than the LDS, keep the plain order.
    int remap0 = -1, remap1 = -1;
    constexpr int kMaxTable = 2 * A_BYTES / 4;  // both A slots
    const bool remapped =
        valid_m <= kMaxTable && (chunk_end - chunk_begin + per_xcd - 1) / per_xcd <= 128;
    if (remapped) {
        int* table = reinterpret_cast<int*>(lds);
        for (int i = tid; i < valid_m; i += NT) {
            const int e = p.expert_ids[i];
            table[i] = e < 0 ? 0x7fffffff : e;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int L = chunk_begin + slot + (lane + 64 * h) * per_xcd;
            int v = -1;
            if (L < chunk_end) {
                const int mt = L / p.n_tiles;
                const int key = table[mt];
                int lo = 0, hi = mt;  // first tile with table == key
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (table[mid] < key) lo = mid + 1;
                    else hi = mid;
                }
                int lo2 = mt + 1, hi2 = valid_m;  // one past its last tile
                while (lo2 < hi2) {
                    const int mid = (lo2 + hi2) >> 1;
                    if (table[mid] <= key) lo2 = mid + 1;
                    else hi2 = mid;
                }
                const int first = lo, count = lo2 - lo;
                const int local = L - first * p.n_tiles;
                v = (first + local % count) * p.n_tiles + local / count;
            }
            if (h == 0) remap0 = v;
            else remap1 = v;
        }
        __syncthreads();  // the table's LDS is the ring's from here on
    }
    auto tile_index = [&](int L) {
        if (!remapped) return L;
        const int k = (L - chunk_begin - slot) / per_xcd;
        return __builtin_amdgcn_readlane(k < 64 ? remap0 : remap1, k & 63);
    };

    // the halves of the A fragments (f = h * FM/2 + i) and the B fragments of one k-step, from
    // per-lane read bases with the wavefront's block offsets folded in, so that the fragment
    // offsets are compile-time constants (immediate offsets of the LDS reads)
    const uint32_t a_rd0 = lds0 + a_off[0] + wm * FM * 2 * kBlk;
    const uint32_t a_rd1 = lds0 + a_off[1] + wm * FM * 2 * kBlk;
    const uint32_t b_rd = lds0 + 2 * A_BYTES + lane * 16 + wn * FN * 2 * kBlk;
    auto read_a_half = [&](int st, int kk, int h, u32x4 (&af)[FM / 2]) {
        const uint32_t ab = (kk ? a_rd1 : a_rd0) + (st & 1) * A_BYTES;
#pragma unroll
        for (int i = 0; i < FM / 2; ++i)
            af[i] = lds_read16(ab + (h * (FM / 2) + i) * 2 * kBlk);
    };
    auto read_b = [&](int st, int kk, u32x4 (&bfr)[FN]) {
        const uint32_t bb = b_rd + (st % NB) * B_BYTES + kk * kBlk;
#pragma unroll
        for (int g = 0; g < FN; ++g) bfr[g] = lds_read16(bb + g * 2 * kBlk);
    };

    f32x4 acc[FM][FN];
    // B-block-major: the fragment refilled last by the previous half-k-step (block FN-1) is
    // consumed last, at least 3 * FM/2 MFMAs after its read was issued
    auto mfma_half = [&](int h, const u32x4 (&af)[FM / 2], const u32x4 (&bfr)[FN]) {
#pragma unroll
        for (int g = 0; g < FN; ++g)
#pragma unroll
            for (int i = 0; i < FM / 2; ++i)
                acc[h * (FM / 2) + i][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(af[i]), as_bf16x8(bfr[g]), acc[h * (FM / 2) + i][g], 0, 0, 0);
    };
    auto mfmas = [&](const u32x4 (&af)[FM], const u32x4 (&bfr)[FN]) {
#pragma unroll
        for (int f = 0; f < FM; ++f)
#pragma unroll
            for (int g = 0; g < FN; ++g)
                acc[f][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(af[f]), as_bf16x8(bfr[g]), acc[f][g], 0, 0, 0);
    };

    int tile = chunk_begin + slot;
    bool pending = false;  // the prologue loads of `tile` are already in flight
    while (tile < chunk_end) {
        if (!pending) {
            fetch(tile_index(tile));
            settle_fetch();
            finish();
            if (expert >= 0) prologue();
        }
        pending = false;
        const int cur_m0 = m0, cur_n = n_tile, cur_expert = expert;
        const int cur_flat = row_flat;
        const int next = tile + per_xcd;

        if (cur_expert < 0) {
            // rows routed to experts outside this rank's map: down writes zeros, gate_up nothing
            if (!GATEUP) {
                for (int idx = tid; idx < BM * (OUTC / 8); idx += NT) {
                    const int row = idx / (OUTC / 8), cc = idx % (OUTC / 8);
                    const int flat = p.sorted_ids[cur_m0 + row];
                    if (flat < p.numel)
                        *reinterpret_cast<u32x4*>(p.C + (int64_t)flat * p.N + cur_n * OUTC +
                                                  cc * 8) = u32x4{0u, 0u, 0u, 0u};
                }
            }
            tile = next;
            continue;
        }

#pragma unroll
        for (int f = 0; f < FM; ++f)
#pragma unroll
            for (int g = 0; g < FN; ++g) acc[f][g] = f32x4{0.f, 0.f, 0.f, 0.f};

        // A 256-row tile whose second half is all padding (an expert's last rows) runs as a
        // half tile: the wavefronts of the second half keep loading and synchronising but do no
        // LDS reads, MFMAs or stores, so each SIMD runs the first-half wavefront alone.
        // Padding rows sit at the end of each expert's segment, so one lookup decides.
        bool active = true;
        if (BM == 256 && wm == 1) active = p.sorted_ids[cur_m0 + 128] < p.numel;

        // Stage pipeline bookkeeping shared by both loops: stage st+1 published (after A(st+1)
        // only B(st+LB) may be pending); the barrier also retires every wavefront's reads of
        // stage st, whose slots the next loads take.
        auto advance = [&](int st) {
            if (st + LB < NST) wait_vmcnt<LPB>();
            else wait_vmcnt<0>();
            barrier_after_lds_reads();
            if (st + 2 < NST) issue_a(st + 2);
            if (st + 1 + LB < NST) issue_b(st + 1 + LB);
        };

        // stage 0 published: only B(LB-1) may still be pending after A(0)
        if (LB - 1 < NST) wait_vmcnt<LPB>();
        else wait_vmcnt<0>();
        barrier_after_lds_reads();
        // down: the routing weight of row `tid`, loaded here (older than every load of the
        // stages below, so their vmcnt accounting is unchanged) and settled after the last stage
        float row_w = 0.0f;
        if (!GATEUP && tid < BM) row_w = p.topk_w[cur_flat < p.numel ? cur_flat : 0];
        if (next < chunk_end) fetch(tile_index(next));
        if (1 < NST) issue_a(1);
        if (LB < NST) issue_b(LB);
        if (!active) {
            for (int st = 0; st + 1 < NST; ++st) advance(st);
        } else if constexpr (FM >= 8) {
            // 256-row tiles (a 128 x 64 block per wavefront): the accumulators take half of the
            // register budget, so A is streamed in halves of FM/2 fragments instead of being
            // double-buffered whole (the first half's MFMAs run while the second half is read,
            // the second half's while the next k-step's first half is read), and B is held as
            // one set that the second half refills fragment by fragment. With two B sets the
            // loop did not fit the 256 registers of a wavefront: the compiler spilled, and each
            // spill reload in the stage loop waited for every outstanding load (vmcnt(0)),
            // draining the ring twice per stage.
            constexpr int FH = FM / 2;
            u32x4 aL[FH], aH[FH], b[FN];
            // second half of a k-step: B-block-major MFMAs, each B fragment replaced by the
            // next k-step's as soon as its last MFMA has issued
            auto mfma_half_refill = [&](const u32x4 (&af)[FH], int st_n, int kk_n) {
#pragma unroll
                for (int g = 0; g < FN; ++g) {
#pragma unroll
                    for (int i = 0; i < FH; ++i)
                        acc[FH + i][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            as_bf16x8(af[i]), as_bf16x8(b[g]), acc[FH + i][g], 0, 0, 0);
                    b[g] = lds_read16(b_rd + (st_n % NB) * B_BYTES + kk_n * kBlk + g * 2 * kBlk);
                }
            };
            read_a_half(0, 0, 0, aL);
            read_b(0, 0, b);
            for (int st = 0; st < NST; ++st) {
                read_a_half(st, 0, 1, aH);
                mfma_half(0, aL, b);
                interleave_reads_mfma<FH, FH * FN>();
                read_a_half(st, 1, 0, aL);
                mfma_half_refill(aH, st, 1);
                refill_sched<FH, FN>();
                read_a_half(st, 1, 1, aH);
                mfma_half(0, aL, b);
                interleave_reads_mfma<FH, FH * FN>();
                if (st + 1 < NST) advance(st);
                read_a_half(st + 1, 0, 0, aL);
                mfma_half_refill(aH, st + 1, 0);
                refill_sched<FH, FN>();
            }
        } else {
            u32x4 a0[FM], b0[FN], a1[FM], b1[FN];
            read_frags(0, 0, a0, b0);
            // One straight-line body per stage (no path split around the last stage) keeps the
            // accumulators in place across iterations; the last stage's read of "stage NST" only
            // touches ring slots no load is writing at that point, and its values are unused.
            for (int st = 0; st < NST; ++st) {
                read_frags(st, 1, a1, b1);
                mfmas(a0, b0);
                interleave_reads_mfma<NR, NM>();
                if (st + 1 < NST) advance(st);
                read_frags(st + 1, 0, a0, b0);
                mfmas(a1, b1);
                interleave_reads_mfma<NR, NM>();
            }
        }

        if (!GATEUP) row_w = settle(cur_flat < p.numel ? row_w : 0.0f);
        if (next < chunk_end) settle_fetch();
        // Every wavefront is done reading the ring: start the next tile's loads, then store.
        barrier_after_lds_reads();
        if (next < chunk_end) {
            finish();
            if (expert >= 0) prologue();
            pending = true;
        }

        // Epilogue, NPASS passes of RP rows through the staging slot: the owners of the pass's
        // rows write them (element i of block (f, g) is row (lane/16)*4 + i, column lane%16;
        // 16-byte chunks XOR-swizzled by row so the four row groups of a write hit different
        // banks), then every lane stores whole 16-byte chunks of rows. Wavefronts of an inactive
        // half tile take part in the barriers; their rows are padding and are never stored.
        const uint32_t stage_lds = lds0 + 2 * A_BYTES + (NB - 1) * B_BYTES;
        auto swz_c = [](int rl) { return ((rl >> 2) & 3) << 2; };
        // down: per-row (assignment, weight) in A slot 1, which the next tile's prologue leaves
        // alone (its A(1) load is issued after that tile's first barrier)
        const uint32_t meta_lds = lds0 + A_BYTES;
        if (!GATEUP) {
            if (tid < BM) {
                *reinterpret_cast<__attribute__((address_space(3))) int*>(meta_lds + tid * 8) = cur_flat;
                *reinterpret_cast<__attribute__((address_space(3))) float*>(meta_lds + tid * 8 + 4) = row_w;
            }
            barrier_after_lds_reads();
        }
#pragma unroll 1
        for (int ps = 0; ps < NPASS; ++ps) {
            if (active) {
#pragma unroll
                for (int f = 0; f < FM; ++f) {
                    const int rb = (wm * FM + f) * 16 - ps * RP;  // block's first staged row
                    if (rb < 0 || rb >= RP) continue;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int rl = rb + (lane >> 4) * 4 + i;
                        const uint32_t rbase = stage_lds + rl * ROWB;
                        float w = 0.0f;
                        if (!GATEUP)
                            w = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
                                meta_lds + (ps * RP + rl) * 8 + 4);
                        if (GATEUP) {
                            // packed w13 interleaves gate block j (2j) with up block j (2j+1)
#pragma unroll
                            for (int pp = 0; pp < FN / 2; ++pp) {
                                const int col = (wn * (FN / 2) + pp) * 16 + (lane & 15);
                                lds_write2(rbase + ((((col >> 3) ^ swz_c(rl)) << 4) | ((col & 7) << 1)),
                                           f32_to_bf16(swiglu_bf16(acc[f][2 * pp][i],
                                                                   acc[f][2 * pp + 1][i])));
                            }
                        } else {
#pragma unroll
                            for (int g = 0; g < FN; ++g) {
                                const int col = (wn * FN + g) * 16 + (lane & 15);
                                lds_write2(rbase + ((((col >> 3) ^ swz_c(rl)) << 4) | ((col & 7) << 1)),
                                           f32_to_bf16(acc[f][g][i] * w));
                            }
                        }
                    }
                }
            }
            barrier_after_lds_reads();
#pragma unroll
            for (int k = 0; k < CPL; ++k) {
                const int c = tid + k * NT, rl = c / CPR, j = c % CPR;
                const u32x4 v = lds_read16(stage_lds + rl * ROWB + ((j ^ swz_c(rl)) << 4));
                if (GATEUP) {
                    const int row = cur_m0 + ps * RP + rl;
                    *reinterpret_cast<u32x4*>(p.C + (int64_t)row * p.N + cur_n * OUTC_C + j * 8) = v;
                } else {
                    const int flat = *reinterpret_cast<const __attribute__((address_space(3))) int*>(
                        meta_lds + (ps * RP + rl) * 8);
                    // the rows are read once, by the k-sum, after this kernel: non-temporal
                    if (flat < p.numel)
                        __builtin_nontemporal_store(
                            v, reinterpret_cast<u32x4*>(p.C + (int64_t)flat * p.N +
                                                         cur_n * OUTC_C + j * 8));
                }
            }
            if (ps + 1 < NPASS) barrier_after_lds_reads();
        }
        tile = next;
    }
    // A prefetched tile is always consumed (`pending` is set only for the tile visited next), so
    // nothing is in flight here; the wait is a guard before the LDS is released.
    wait_vmcnt<0>();
}

// Per-device launch state: the CU count, and whether a kernel's dynamic-LDS limit has been raised
// on that device (done once, under a lock, before the first launch there).
constexpr int kMaxDevices = 64;

int current_device() {
    int dev = 0;
    return hipGetDevice(&dev) == hipSuccess ? dev : 0;
}

int cu_count() {
    static std::atomic<int> cus[kMaxDevices];
    const int dev = current_device();
    int n = dev < kMaxDevices ? cus[dev].load(std::memory_order_relaxed) : 0;
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
        n = 256;
    if (dev < kMaxDevices) cus[dev].store(n, std::memory_order_relaxed);
    return n;
}

// done[] belongs to one kernel (each launch_tile instantiation passes its own).
void raise_lds_limit(const void* kernel, size_t lds, std::atomic<bool> (&done)[kMaxDevices]) {
    static std::mutex mu;
    const int dev = current_device();
    if (dev < kMaxDevices && done[dev].load(std::memory_order_acquire)) return;
    std::lock_guard<std::mutex> lock(mu);
    if (dev < kMaxDevices && done[dev].load(std::memory_order_relaxed)) return;
    (void)hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (dev < kMaxDevices) done[dev].store(true, std::memory_order_release);
}

template <int BM, bool GATEUP>
void launch_tile(GemmArgs g, hipStream_t stream) {
    constexpr int WM = BM >= 128 ? 2 : 1;
    constexpr int a_bytes = BM / 8 * kBlk, b_bytes = 2 * (kBN / 16) * kBlk;
    constexpr int NB = (160 * 1024 - 2 * a_bytes) / b_bytes > 4 ? 4
                                                                 : (160 * 1024 - 2 * a_bytes) / b_bytes;
    const size_t lds = (size_t)2 * a_bytes + (size_t)NB * b_bytes;
    static std::atomic<bool> lds_raised[kMaxDevices];
    raise_lds_limit((const void*)moe_tile_kernel<BM, GATEUP, WM, NB>, lds, lds_raised);
    // persistent: at most one workgroup per CU, a multiple of 8 so every XCD gets the same count
    const int64_t tiles = (int64_t)g.m_tiles * g.n_tiles;
    int64_t grid = tiles < cu_count() ? tiles : cu_count();
    grid = (grid + 7) / 8 * 8;
    hipLaunchKernelGGL((moe_tile_kernel<BM, GATEUP, WM, NB>), dim3((unsigned)grid),
                       dim3(64 * kNW), lds, stream, g);
}

}  // namespace

// Packed weights only; K % 64 == 0; gate_up: 2N % 256 == 0; down: N % 256 == 0.
bool tile_kernels_take(int H, int I) {
    return H % 64 == 0 && (2 * I) % kBN == 0 && I % 64 == 0 && H % kBN == 0;
}

bool tile256_takes_x(int64_t T, int K) { return T * (int64_t)K * 2 < (1ll << 32); }

bool launch_tile_gate_up(GemmArgs g, int block_m, hipStream_t stream) {
    if (g.K % 64 != 0 || (2 * g.N) % kBN != 0) return false;
    // the 256-row kernel gathers x rows through 32-bit byte offsets
    if (block_m == 256 && !tile256_takes_x((g.numel + g.top_k - 1) / g.top_k, g.K)) return false;
    g.n_tiles = 2 * g.N / kBN;
    if (block_m == 256) launch_tile<256, true>(g, stream);
    else if (block_m == 128) launch_tile<128, true>(g, stream);
    else if (block_m == 64) launch_tile<64, true>(g, stream);
    else return false;
    return true;
}

bool launch_tile_down(GemmArgs g, int block_m, hipStream_t stream) {
    if (g.K % 64 != 0 || g.N % kBN != 0) return false;
    g.n_tiles = g.N / kBN;
    if (block_m == 256) launch_tile<256, false>(g, stream);
    else if (block_m == 128) launch_tile<128, false>(g, stream);
    else if (block_m == 64) launch_tile<64, false>(g, stream);
    else return false;
    return true;
}

}  // namespace tsm
