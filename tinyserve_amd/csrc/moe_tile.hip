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

// The compiler does not order LDS reads after the global->LDS loads that fill them, and
// __syncthreads() would drain every outstanding load (a release fence) before each barrier. The
// ring is therefore synchronised by hand: each wavefront waits (vmcnt) for its own loads of the
// stage it is about to read and for its own LDS reads of the previous stage (lgkmcnt), then a
// plain s_barrier publishes the stage to every wavefront and frees the slot the next loads
// overwrite. The asm statements carry "memory" clobbers so no LDS access moves across them.
__device__ __forceinline__ u32x4 lds_read16(uint32_t addr) {
    return *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(addr);
}
__device__ __forceinline__ void barrier_after_lds_reads() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int kBN = 256;     // B rows per tile
constexpr int kBlk = 1024;   // bytes per 16x32 operand block


// kStageK: MFMA k-steps (of 32) per pipeline stage; kStages: LDS ring depth (kStages - 1 stages
// of loads in flight while one is consumed); NW: wavefronts (2 x NW/2 grid over the tile).
template <int BM, bool GATEUP, int kStageK, int kStages, int NW>
__global__ __launch_bounds__(64 * NW, 2) void moe_tile_kernel(GemmArgs p) {
    constexpr int NT = 64 * NW;
    constexpr int WN = NW / 2;              // wavefront columns
    constexpr int MB = BM / 16;             // A row blocks per tile
    constexpr int NBK = kBN / 16;           // B row blocks per tile (16)
    constexpr int A_BLKS = MB * kStageK;    // A blocks per stage
    constexpr int B_BLKS = NBK * kStageK;   // B blocks per stage
    constexpr int NBLK = A_BLKS + B_BLKS;
    constexpr int STAGE_BYTES = NBLK * kBlk;
    constexpr int LPW = (NBLK + NW - 1) / NW;  // load slots per wavefront per stage
    constexpr int FM = MB / 2;              // A blocks per wavefront (rows BM/2)
    constexpr int FN = NBK / WN;            // B blocks per wavefront
    static_assert(!GATEUP || FN % 2 == 0, "gate/up block pairs per wavefront");
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
            for (int idx = tid; idx < BM * (OUTC / 8); idx += NT) {
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

    // Load slots: wavefront w loads blocks w, w + NW, ... of every stage (A blocks first, then B),
    // each lane the 16 bytes it will read back from LDS. A block (row block mb, k-step kk): the
    // lane's gathered row at column 32*kk + 8*q; B block: 16-row block nb of the packed weights.
    const bf16_t* src[LPW];
    int stride[LPW];   // elements per stage
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
        const int b = wave + j * NW;
        src[j] = nullptr;
        stride[j] = 0;
        if (b < A_BLKS) {
            const int mb = b / kStageK, kk = b % kStageK;
            const int row = m0 + mb * 16 + r;
            int64_t src_row;
            if (GATEUP) {
                int flat = p.sorted_ids[row];
                if (flat >= p.numel) flat = 0;  // padding row: any valid row, result discarded
                src_row = flat / p.top_k;
            } else {
                src_row = row;
            }
            src[j] = p.A + src_row * p.K + kk * 32 + q * 8;
            stride[j] = kStageK * 32;
        } else if (b < NBLK) {
            const int nb = (b - A_BLKS) / kStageK, kk = (b - A_BLKS) % kStageK;
            const bf16_t* Be = p.B + (int64_t)expert * (GATEUP ? 2 : 1) * p.N * p.K;
            src[j] = Be + ((int64_t)(n_tile * NBK + nb) * KS + kk) * 512 + lane * 8;
            stride[j] = kStageK * 512;
        }
    }
    auto issue = [&](int st) {
        char* base = lds + (st % kStages) * STAGE_BYTES;
#pragma unroll
        for (int j = 0; j < LPW; ++j) {
            const int b = wave + j * NW;
            if (NBLK % NW == 0 || b < NBLK)
                __builtin_amdgcn_global_load_lds((const void*)(src[j] + (int64_t)st * stride[j]),
                                                 (lds_void*)(base + b * kBlk), 16, 0, 0);
        }
    };
    // LDS slot of A block (mb, kk): mb*kStageK + kk; of B block (nb, kk): A_BLKS + nb*kStageK+kk

    const int wm = wave / WN, wn = wave % WN;
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

    // Loads issued per wavefront per stage (slots beyond NBLK issue nothing).
    constexpr int LPS = (NBLK % NW == 0) ? LPW : -1;
    static_assert(LPS > 0, "stage blocks must split evenly over the wavefronts");
    constexpr int NPRE = kStages - 1;              // stages in flight ahead of the one read
#pragma unroll
    for (int st = 0; st < NPRE; ++st)
        if (st < NST) issue(st);
    for (int st = 0; st < NST; ++st) {
        // this wavefront's loads for stage st are done once only the later stages it has issued
        // are pending; the barrier then publishes every wavefront's share of stage st and
        // retires the reads of st - 1, whose slot the next issue overwrites
        const int later = min(NPRE - 1, NST - 1 - st);
        if (later >= NPRE - 1) wait_vmcnt<LPS * (NPRE - 1)>();
        else if (NPRE >= 3 && later == 1) wait_vmcnt<LPS>();
        else if (NPRE >= 4 && later == 2) wait_vmcnt<(NPRE >= 4 ? LPS * 2 : 0)>();
        else if (NPRE >= 5 && later == 3) wait_vmcnt<(NPRE >= 5 ? LPS * 3 : 0)>();
        else wait_vmcnt<0>();
        barrier_after_lds_reads();
        if (st + NPRE < NST) issue(st + NPRE);
#pragma unroll
        for (int kk = 0; kk < kStageK; ++kk) {
            u32x4 af[FM], bfr[FN];
            read_frags(st, kk, af, bfr);
            mfmas(af, bfr);
        }
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
    constexpr int NW = BM >= 128 ? 8 : 4;                       // wavefronts per workgroup
    constexpr int SK = ((BM / 16 + kBN / 16) % NW == 0) ? 1 : 2;  // k-steps per stage
    constexpr int stage = (BM / 16 + kBN / 16) * SK * kBlk;     // bytes per stage
    constexpr int NS = (80 * 1024) / stage > 6 ? 6 : (80 * 1024) / stage;  // ring depth, 2 WG/CU
    const size_t lds = (size_t)NS * stage;
    static bool configured = false;
    if (!configured) {
        (void)hipFuncSetAttribute((const void*)moe_tile_kernel<BM, GATEUP, SK, NS, NW>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        configured = true;
    }
    hipLaunchKernelGGL((moe_tile_kernel<BM, GATEUP, SK, NS, NW>), dim3(g.m_tiles * g.n_tiles),
                       dim3(64 * NW), lds, stream, g);
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
