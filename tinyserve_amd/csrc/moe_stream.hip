// Weight-streaming grouped GEMMs for decode-sized batches (16-row expert tiles).
//
// At decode sizes each expert sees a handful of rows, so the layer is a stream of expert weights
// (768 MiB gate_up + 384 MiB down for Qwen3-30B-A3B) and the kernel's job is to keep HBM busy.
// Design:
//   - one workgroup = one 16-row expert tile x NB 16-row blocks of B, 4 wavefronts splitting K
//     (split-K inside the workgroup, partials summed through LDS in fixed wavefront order);
//   - every operand goes straight from global memory into MFMA registers (no LDS staging) and all
//     S*(1+NB) loads of a wavefront are issued before its first MFMA;
//   - B comes either in the reference layout ([N, K] rows: one load instruction covers 16 rows x
//     64 bytes) or in the MFMA-tiled layout of moe_pack.hip (one load instruction covers 1 KiB of
//     contiguous memory);
//   - 16x16x32 bf16 MFMA, fp32 accumulation; epilogues with the reference's rounding points
//     (SwiGLU on bf16-rounded gate/up, bf16-rounded silu; down output scaled by the fp32 routing
//     weight, then rounded, scattered to assignment order).
// Reference: the _fused_moe_kernel computation (tinykernels.py:1589-1765) at BLOCK_M=16.
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

// S: MFMA k-steps per wavefront (K = 4 * 32 * S). NB: 16-row B blocks per wavefront; for gate_up
// NB = 2 (one gate block and the matching up block -> 16 activation columns). WN: groups of 4
// wavefronts, each group taking the next NB blocks (down GEMM only).
template <int S, int NB, int WN, bool GATEUP, bool PACKED>
__global__ __launch_bounds__(256 * WN, 2 / WN) void moe_stream_kernel(GemmArgs p) {
    static_assert(!GATEUP || WN == 1, "gate_up uses one wavefront group");
    constexpr int BM = 16;
    constexpr int NT = 256 * WN;                      // threads
    constexpr int OUTC = GATEUP ? 16 : 16 * NB * WN;  // output columns per workgroup
    __shared__ f32x4 red[4][WN * NB][64];

    const int G = p.m_tiles * p.n_tiles;
    const int pid = blockIdx.x;
    const int xcd = pid & 7, q8 = G >> 3, r8 = G & 7;
    const int logical = xcd * q8 + min(xcd, r8) + (pid >> 3);
    const int m_tile = logical % p.m_tiles, n_tile = logical / p.m_tiles;
    const int m0 = m_tile * BM;
    if (m0 >= p.total[0]) return;
    const int expert = p.expert_ids[m_tile];
    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3, wgrp = tid >> 8;

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
    const int kbase = wave * (32 * S) + q * 8;  // this lane's first k; step s adds 32*s
    const bf16_t* Be = p.B + (int64_t)expert * (GATEUP ? 2 : 1) * p.N * p.K;

    u32x4 b[NB][S];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const u32x4* src;
        int stride;  // in 16-byte units between consecutive k-steps
        if (PACKED) {
            const int blk = GATEUP ? 2 * n_tile + nb : (n_tile * WN + wgrp) * NB + nb;
            src = reinterpret_cast<const u32x4*>(
                      Be + ((int64_t)blk * (p.K / 32) + wave * S) * 512) + lane;
            stride = 64;
        } else {
            const int row = GATEUP ? (nb == 0 ? 0 : p.N) + n_tile * 16 + r
                                   : n_tile * OUTC + (wgrp * NB + nb) * 16 + r;
            src = reinterpret_cast<const u32x4*>(Be + (int64_t)row * p.K + kbase);
            stride = 4;
        }
#pragma unroll
        for (int s = 0; s < S; ++s) b[nb][s] = __builtin_nontemporal_load(src + stride * s);
    }
    const bf16_t* a_src;
    if (GATEUP) {
        const int flat = p.sorted_ids[m0 + r];
        a_src = flat < p.numel ? p.A + (int64_t)(flat / p.top_k) * p.K + kbase : nullptr;
    } else {
        a_src = p.A + (int64_t)(m0 + r) * p.K + kbase;
    }
    u32x4 a[S];
    if (a_src) {
        const u32x4* src = reinterpret_cast<const u32x4*>(a_src);
#pragma unroll
        for (int s = 0; s < S; ++s) a[s] = src[4 * s];
    } else {
#pragma unroll
        for (int s = 0; s < S; ++s) a[s] = u32x4{0u, 0u, 0u, 0u};
    }

    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[s]), as_bf16x8(b[nb][s]),
                                                              acc[nb], 0, 0, 0);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) red[wave][wgrp * NB + nb][lane] = acc[nb];
    __syncthreads();

    // Thread (lane l, element i, group g) finalises row (l/16)*4 + i, column l%16 of the blocks
    // of group g, summing the four K-quarter partials in fixed order.
    const int l = tid & 63, i = (tid >> 6) & 3;
    const int row = (l >> 4) * 4 + i, col = l & 15;
    float v[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int bb = wgrp * NB + nb;
        v[nb] = ((red[0][bb][l][i] + red[1][bb][l][i]) + red[2][bb][l][i]) + red[3][bb][l][i];
    }
    if (GATEUP) {
        p.C[(int64_t)(m0 + row) * p.N + n_tile * 16 + col] = f32_to_bf16(swiglu_bf16(v[0], v[1]));
    } else {
        const int flat = p.sorted_ids[m0 + row];
        if (flat < p.numel) {
            const float w = p.topk_w[flat];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                p.C[(int64_t)flat * p.N + n_tile * OUTC + (wgrp * NB + nb) * 16 + col] =
                    f32_to_bf16(v[nb] * w);
        }
    }
}

template <int S, int NB, bool GATEUP, bool PACKED, int WN = 1>
void launch_s(const GemmArgs& g, hipStream_t stream) {
    hipLaunchKernelGGL((moe_stream_kernel<S, NB, WN, GATEUP, PACKED>),
                       dim3(g.m_tiles * g.n_tiles), dim3(256 * WN), 0, stream, g);
}

template <bool PACKED>
bool gate_up_s(const GemmArgs& g, hipStream_t stream) {
    switch (g.K / 128) {
        case 2: launch_s<2, 2, true, PACKED>(g, stream); return true;
        case 4: launch_s<4, 2, true, PACKED>(g, stream); return true;
        case 6: launch_s<6, 2, true, PACKED>(g, stream); return true;
        case 8: launch_s<8, 2, true, PACKED>(g, stream); return true;
        case 12: launch_s<12, 2, true, PACKED>(g, stream); return true;
        case 16: launch_s<16, 2, true, PACKED>(g, stream); return true;
        default: return false;
    }
}

// Down GEMM: two groups of four wavefronts, four 16-column blocks each (128 columns per
// workgroup) when the K slice is short (register budget); two blocks, one group otherwise.
template <bool PACKED>
bool down_s(GemmArgs g, hipStream_t stream) {
    const int S = g.K / 128;
    if (S <= 8 && g.N % 128 == 0) {
        g.n_tiles = g.N / 128;
        switch (S) {
            case 2: launch_s<2, 4, false, PACKED, 2>(g, stream); return true;
            case 4: launch_s<4, 4, false, PACKED, 2>(g, stream); return true;
            case 6: launch_s<6, 4, false, PACKED, 2>(g, stream); return true;
            case 8: launch_s<8, 4, false, PACKED, 2>(g, stream); return true;
            default: return false;
        }
    }
    if (g.N % 32 != 0) return false;
    g.n_tiles = g.N / 32;
    switch (S) {
        case 12: launch_s<12, 2, false, PACKED>(g, stream); return true;
        case 16: launch_s<16, 2, false, PACKED>(g, stream); return true;
        default: return false;
    }
}

}  // namespace

// g.N / g.K / pointers filled by the caller; m_tiles set for 16-row tiles; n_tiles set here.
bool launch_stream_gate_up(GemmArgs g, bool packed, hipStream_t stream) {
    if (g.N % 16 != 0 || g.K % 128 != 0) return false;
    g.n_tiles = g.N / 16;
    return packed ? gate_up_s<true>(g, stream) : gate_up_s<false>(g, stream);
}

bool launch_stream_down(GemmArgs g, bool packed, hipStream_t stream) {
    if (g.K % 128 != 0) return false;
    return packed ? down_s<true>(g, stream) : down_s<false>(g, stream);
}

}  // namespace tsm
