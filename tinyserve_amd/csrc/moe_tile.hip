// LDS-pipelined grouped GEMMs for prefill-sized batches (64/128-row expert tiles).
//
// Workgroup tile: BM expert-sorted rows x 256 rows of B (gate_up: 8 gate + 8 up 16-row blocks ->
// 128 activation columns; down: 256 output columns), 4 wavefronts in a 2 x 2 grid, each owning a
// (BM/2) x 128 block of C in 16x16x32 bf16 MFMA accumulators.
//
// Operands reach LDS through direct global->LDS loads (global_load_lds_dwordx4: 64 lanes x 16 B,
// written to LDS in lane order), so LDS holds every 16-row x 32-k operand block in exactly the
// order an MFMA lane reads it (ds_read_b128 at lane*16, no bank conflicts, no register staging):
//   - B comes from the MFMA-tiled (packed) weights, where such a block is 1 KiB of contiguous
//     memory;
//   - A rows are gathered per lane (gate_up: x[sorted_id / top_k]; down: activation rows), each
//     lane fetching the 16 bytes it will later read back.
// K is consumed in stages of 64 (two MFMA k-steps) through a 3-deep LDS ring: the loads of stage
// s+2 are issued before stage s is computed.
// Reference computation: _fused_moe_kernel (tinykernels.py:1589-1765), epilogues as in the
// weight-streaming kernels (SwiGLU with the reference's bf16 rounding points; routing-weight
// scaling and scatter to assignment order).
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ float swiglu_tile(float g, float u) {
    g = round_bf16(g);
    u = round_bf16(u);
    const float s = round_bf16(g / (1.0f + __expf(-g)));
    return s * u;
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt in bits 3:0
// and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS reads as inline assembly: the compiler's wait-count pass cannot see that the ring slot
// being read is not the one the in-flight global->LDS loads target and would otherwise drain all
// loads before every read. Completion is tracked by hand (wait_vmcnt before the barrier that
// publishes a stage; lgkmcnt(0) before the MFMAs that consume a read).
__device__ __forceinline__ u32x4 lds_read16(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
    return v;
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void barrier_nofence() { asm volatile("s_barrier" ::: "memory"); }

constexpr int kStageK = 2;   // MFMA k-steps (of 32) per pipeline stage
constexpr int kStages = 3;   // LDS ring depth
constexpr int kBN = 256;     // B rows per tile
constexpr int kBlk = 1024;   // bytes per 16x32 operand block

template <int BM, bool GATEUP>
__global__ __launch_bounds__(256, 1) void moe_tile_kernel(GemmArgs p) {
    constexpr int MB = BM / 16;             // A row blocks per tile
    constexpr int NBK = kBN / 16;           // B row blocks per tile (16)
    constexpr int A_BLKS = MB * kStageK;    // A blocks per stage
    constexpr int B_BLKS = NBK * kStageK;   // B blocks per stage
    constexpr int STAGE_BYTES = (A_BLKS + B_BLKS) * kBlk;
    constexpr int A_PER_WAVE = A_BLKS / 4, B_PER_WAVE = B_BLKS / 4;
    constexpr int FM = MB / 2;              // A blocks per wavefront (rows BM/2)
    constexpr int FN = NBK / 2;             // B blocks per wavefront (8)
    static_assert(A_BLKS % 4 == 0 && B_BLKS % 4 == 0, "even split of loads over wavefronts");
    extern __shared__ __attribute__((aligned(1024))) char lds[];

    const int G = p.m_tiles * p.n_tiles;
    const int pid = blockIdx.x;
    const int xcd = pid & 7, q8 = G >> 3, r8 = G & 7;
    const int logical = xcd * q8 + min(xcd, r8) + (pid >> 3);
    const int m_tile = logical % p.m_tiles, n_tile = logical / p.m_tiles;
    const int m0 = m_tile * BM;
    if (m0 >= p.total[0]) return;
    const int expert = p.expert_ids[m_tile];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int OUTC = GATEUP ? kBN / 2 : kBN;

    if (expert < 0) {
        if (!GATEUP) {
            for (int idx = tid; idx < BM * (OUTC / 8); idx += 256) {
                const int row = idx / (OUTC / 8), cc = idx % (OUTC / 8);
                const int flat = p.sorted_ids[m0 + row];
                if (flat < p.numel)
                    *reinterpret_cast<u32x4*>(p.C + (int64_t)flat * p.N + n_tile * OUTC +
                                              cc * 8) = u32x4{0u, 0u, 0u, 0u};
            }
        }
        return;
    }

    const int r = lane & 15, q = lane >> 4;
    const int KS = p.K / 32;                 // k-steps
    const int NST = KS / kStageK;            // stages

    // Per-lane global sources. A: this wavefront loads row blocks mb = wave*A_PER_WAVE/kStageK..
    // (each for kStageK k-steps); the lane's row and 16-byte column inside the 16x32 block.
    constexpr int AMB = A_PER_WAVE / kStageK;  // A row blocks loaded per wavefront
    const bf16_t* a_row[AMB > 0 ? AMB : 1];
#pragma unroll
    for (int j = 0; j < AMB; ++j) {
        const int row = m0 + (wave * AMB + j) * 16 + r;
        int64_t src_row;
        if (GATEUP) {
            int flat = p.sorted_ids[row];
            if (flat >= p.numel) flat = 0;  // padding row: any valid row, result discarded
            src_row = flat / p.top_k;
        } else {
            src_row = row;
        }
        a_row[j] = p.A + src_row * p.K + q * 8;
    }
    // B: this wavefront loads n-blocks wave*BNB.. of the tile, all kStageK k-steps.
    constexpr int BNB = B_PER_WAVE / kStageK;
    const bf16_t* Be = p.B + (int64_t)expert * (GATEUP ? 2 : 1) * p.N * p.K;
    const bf16_t* b_blk = Be + ((int64_t)(n_tile * NBK + wave * BNB) * KS) * 512 + lane * 8;

    auto issue = [&](int st) {
        char* base = lds + (st % kStages) * STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < AMB; ++j)
#pragma unroll
            for (int kk = 0; kk < kStageK; ++kk) {
                const int blk = (wave * AMB + j) * kStageK + kk;
                __builtin_amdgcn_global_load_lds(
                    (const void*)(a_row[j] + (st * kStageK + kk) * 32),
                    (lds_void*)(base + blk * kBlk), 16, 0, 0);
            }
#pragma unroll
        for (int j = 0; j < BNB; ++j)
#pragma unroll
            for (int kk = 0; kk < kStageK; ++kk) {
                const int blk = A_BLKS + (wave * BNB + j) * kStageK + kk;
                __builtin_amdgcn_global_load_lds(
                    (const void*)(b_blk + ((int64_t)j * KS + st * kStageK + kk) * 512),
                    (lds_void*)(base + blk * kBlk), 16, 0, 0);
            }
    };

    const int wm = wave >> 1, wn = wave & 1;
    f32x4 acc[FM][FN];
#pragma unroll
    for (int f = 0; f < FM; ++f)
#pragma unroll
        for (int g = 0; g < FN; ++g) acc[f][g] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t lds_lane =
        (uint32_t)(uintptr_t)(lds_void*)lds + (uint32_t)lane * 16;  // LDS byte address
    auto read_frags = [&](int st, int kk, u32x4 (&af)[FM], u32x4 (&bfr)[FN]) {
        const uint32_t base = lds_lane + (st % kStages) * STAGE_BYTES;
#pragma unroll
        for (int f = 0; f < FM; ++f)
            af[f] = lds_read16(base + ((wm * FM + f) * kStageK + kk) * kBlk);
#pragma unroll
        for (int g = 0; g < FN; ++g)
            bfr[g] = lds_read16(base + (A_BLKS + (wn * FN + g) * kStageK + kk) * kBlk);
    };
    auto mfmas = [&](const u32x4 (&af)[FM], const u32x4 (&bfr)[FN]) {
#pragma unroll
        for (int f = 0; f < FM; ++f)
#pragma unroll
            for (int g = 0; g < FN; ++g)
                acc[f][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(af[f]), as_bf16x8(bfr[g]), acc[f][g], 0, 0, 0);
    };

    issue(0);
    if (NST > 1) issue(1);
    for (int st = 0; st < NST; ++st) {
        // this wavefront's loads for stage st are done once at most one later stage is pending;
        // the barrier then publishes every wavefront's share and retires the reads of st - 1
        if (st + 1 < NST)
            wait_vmcnt<A_PER_WAVE + B_PER_WAVE>();
        else
            wait_vmcnt<0>();
        barrier_nofence();
        if (st + 2 < NST) issue(st + 2);
        static_assert(kStageK == 2, "two k-steps per stage");
        u32x4 a0[FM], b0[FN], a1[FM], b1[FN];
        read_frags(st, 0, a0, b0);
        wait_lgkm0();
        read_frags(st, 1, a1, b1);
        mfmas(a0, b0);
        wait_lgkm0();
        mfmas(a1, b1);
    }

    // Epilogue: element i of block (f, g) is row (lane/16)*4 + i, column lane%16.
#pragma unroll
    for (int f = 0; f < FM; ++f) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = m0 + (wm * FM + f) * 16 + (lane >> 4) * 4 + i;
            if (GATEUP) {
                // packed w13 interleaves gate block j (2j) with up block j (2j+1)
#pragma unroll
                for (int pp = 0; pp < FN / 2; ++pp) {
                    const int col = (n_tile * (NBK / 2) + wn * (FN / 2) + pp) * 16 + (lane & 15);
                    p.C[(int64_t)row * p.N + col] =
                        f32_to_bf16(swiglu_tile(acc[f][2 * pp][i], acc[f][2 * pp + 1][i]));
                }
            } else {
                const int flat = p.sorted_ids[row];
                if (flat < p.numel) {
                    const float w = p.topk_w[flat];
#pragma unroll
                    for (int g = 0; g < FN; ++g) {
                        const int col = (n_tile * NBK + wn * FN + g) * 16 + (lane & 15);
                        p.C[(int64_t)flat * p.N + col] = f32_to_bf16(acc[f][g][i] * w);
                    }
                }
            }
        }
    }
}

template <int BM, bool GATEUP>
void launch_tile(GemmArgs g, hipStream_t stream) {
    constexpr int stage = (BM / 16 + kBN / 16) * kStageK * kBlk;
    const size_t lds = (size_t)kStages * stage;
    static bool configured = false;
    if (!configured) {
        (void)hipFuncSetAttribute((const void*)moe_tile_kernel<BM, GATEUP>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        configured = true;
    }
    hipLaunchKernelGGL((moe_tile_kernel<BM, GATEUP>), dim3(g.m_tiles * g.n_tiles), dim3(256), lds,
                       stream, g);
}

}  // namespace

// Packed weights only; K % 64 == 0; gate_up: 2N % 256 == 0; down: N % 256 == 0.
bool launch_tile_gate_up(GemmArgs g, int block_m, hipStream_t stream) {
    if (g.K % 64 != 0 || (2 * g.N) % kBN != 0) return false;
    g.n_tiles = 2 * g.N / kBN;
    if (block_m == 128) launch_tile<128, true>(g, stream);
    else if (block_m == 64) launch_tile<64, true>(g, stream);
    else return false;
    return true;
}

bool launch_tile_down(GemmArgs g, int block_m, hipStream_t stream) {
    if (g.K % 64 != 0 || g.N % kBN != 0) return false;
    g.n_tiles = g.N / kBN;
    if (block_m == 128) launch_tile<128, false>(g, stream);
    else if (block_m == 64) launch_tile<64, false>(g, stream);
    else return false;
    return true;
}

}  // namespace tsm
