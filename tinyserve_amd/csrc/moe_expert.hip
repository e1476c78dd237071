// Expert-major weight-streaming GEMMs for decode-sized batches: no separate permutation step.
//
// One workgroup owns (expert e, a narrow block of output columns). It first scans the routing
// ids (a few KiB, L2-resident): an LDS histogram of all experts gives e's first row in the
// compact expert-sorted activation buffer (the exclusive prefix of the counts), and a ballot
// compaction gives e's assignments in increasing flat index (the same stable order as
// moe_align_block_size, tinykernels.py:1070-1190). Experts with no assignment exit before
// touching their weights. It then streams its weight block straight into MFMA registers (all
// loads issued before the first MFMA; packed layout = 1 KiB contiguous per load instruction) and
// runs 16-row sub-tiles of its assignments against the resident weights, so each expert's
// weights are read exactly once per layer whatever its row count. K is split over the four
// wavefronts of a group, partials are summed through LDS in fixed order.
//
// gate_up: act[start_e + j, :] = SwiGLU(x[flat_j / k] @ W1/W3^T) (reference rounding points).
// down:    rows[flat_j, :] = bf16((act[start_e + j] @ W2^T) * topk_w[flat_j]); the extra expert
//          index E zero-fills the rows of assignments owned by another GPU (ids outside [0, E)).
// Reference computation: _fused_moe_kernel (tinykernels.py:1589-1765).
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

constexpr int kMaxBucketsE = 513;

// MODE 0: workgroup column = expert index; 1: the same, with the weights requested before the
// id scan (most experts have rows); 2 (compact, few assignments): workgroup column j takes the
// j-th non-empty bucket of the ids, so the grid spans min(numel, experts) columns, not all E.
template <int S, int NB, int WN, bool GATEUP, bool PACKED, int MODE>
__global__ __launch_bounds__(256 * WN, 2) void moe_expert_kernel(ExpertArgs p) {
    constexpr bool SPEC = MODE == 1, COMPACT = MODE == 2;
    static_assert(!GATEUP || NB == 2, "gate_up: one gate and one up block per wavefront group");
    constexpr int NT = 256 * WN;
    constexpr int OUTC = GATEUP ? 16 * WN : 16 * NB * WN;  // output columns per workgroup
    __shared__ f32x4 red[4][WN * NB][64];
    __shared__ int s_hist[kMaxBucketsE];
    __shared__ int s_rows[kExpertMaxRows];
    __shared__ int s_wsum[NT / 64];
    __shared__ int s_start;
    __shared__ int s_expert;

    const int col = blockIdx.x / p.n_tiles, n_tile = blockIdx.x % p.n_tiles;
    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3, wgrp = tid >> 8;
    const int wid = tid >> 6;
    int e = col;

    // 1. scan the ids: histogram (for e's start) and e's assignments in flat order. The ids
    // (at most kIdRegs per thread) are requested before the weights so their loads return first.
    constexpr int kIdRegs = kExpertMaxRows / NT;
    int idr[kIdRegs];
#pragma unroll
    for (int c = 0; c < kIdRegs; ++c) {
        const int64_t i = (int64_t)c * NT + tid;
        idr[c] = i < p.numel ? p.ids[i] : -2;
    }
    // this expert's weight block into registers, requested before the id scan when most experts
    // are expected to have rows (SPEC), after it otherwise (empty experts then cost no weights)
    const int r = lane & 15, q = lane >> 4;
    const int kbase = wave * (32 * S) + q * 8;  // this lane's first k; step s adds 32*s
    u32x4 b[NB][S];
    auto load_b = [&]() {
        const bf16_t* Be = p.B + (int64_t)e * (GATEUP ? 2 : 1) * p.N * p.K;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const u32x4* src;
            int stride;
            if (PACKED) {
                const int blk = (n_tile * WN + wgrp) * NB + nb;  // gate_up: gate 2c, up 2c+1
                src = reinterpret_cast<const u32x4*>(
                          Be + ((int64_t)blk * (p.K / 32) + wave * S) * 512) + lane;
                stride = 64;
            } else {
                const int row = GATEUP ? (nb == 0 ? 0 : p.N) + (n_tile * WN + wgrp) * 16 + r
                                       : n_tile * OUTC + (wgrp * NB + nb) * 16 + r;
                src = reinterpret_cast<const u32x4*>(Be + (int64_t)row * p.K + kbase);
                stride = 4;
            }
#pragma unroll
            for (int s = 0; s < S; ++s) b[nb][s] = __builtin_nontemporal_load(src + stride * s);
        }
    };
    if (SPEC && e != p.E) load_b();

    for (int bk = tid; bk <= p.E; bk += NT) s_hist[bk] = 0;
    __syncthreads();
    if (COMPACT) {
        // histogram first, then this column's bucket: the col-th non-empty one in order
        // (0..E-1 for gate_up; 0..E for down, E being the remote bucket)
#pragma unroll
        for (int c = 0; c < kIdRegs; ++c) {
            if ((int64_t)c * NT >= p.numel) break;
            const int64_t i = (int64_t)c * NT + tid;
            if (i < p.numel) {
                const int id = idr[c];
                atomicAdd(&s_hist[(id >= 0 && id < p.E) ? id : p.E], 1);
            }
        }
        __syncthreads();
        if (wid == 0) {
            const int nb_all = GATEUP ? p.E : p.E + 1;
            int seen = 0, found = -1;
            for (int base = 0; base < nb_all && found < 0; base += 64) {
                const bool nz = base + lane < nb_all && s_hist[base + lane] > 0;
                const uint64_t bal = __ballot(nz);
                const int n = __popcll(bal);
                if (col < seen + n) {
                    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
                    if (nz && seen + (int)__popcll(bal & lt) == col) s_expert = base + lane;
                    found = 1;
                }
                seen += n;
            }
            if (found < 0 && lane == 0) s_expert = -1;
        }
        __syncthreads();
        e = s_expert;
        if (e < 0) return;  // fewer non-empty buckets than columns
    }
    const bool remote = (e == p.E);
    int count = 0;
#pragma unroll
    for (int c = 0; c < kIdRegs; ++c) {
        if ((int64_t)c * NT >= p.numel) break;
        const int64_t i = (int64_t)c * NT + tid;
        const int id = idr[c];
        const bool in = i < p.numel;
        if (!COMPACT && in) atomicAdd(&s_hist[(id >= 0 && id < p.E) ? id : p.E], 1);
        const bool match = in && (remote ? (id < 0 || id >= p.E) : id == e);
        const uint64_t bal = __ballot(match);
        const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        if (lane == 0) s_wsum[wid] = __popcll(bal);
        __syncthreads();
        int off = count;
        for (int w = 0; w < wid; ++w) off += s_wsum[w];
        if (match) s_rows[off + __popcll(bal & lt)] = (int)i;
        for (int w = 0; w < NT / 64; ++w) count += s_wsum[w];
        __syncthreads();
    }
    if (count == 0) return;

    if (remote) {  // down only: zero rows of assignments owned by another GPU
        for (int idx = tid; idx < count * (OUTC / 8); idx += NT) {
            const int j = idx / (OUTC / 8), cc = idx % (OUTC / 8);
            *reinterpret_cast<u32x4*>(p.C + (int64_t)s_rows[j] * p.N + n_tile * OUTC + cc * 8) =
                u32x4{0u, 0u, 0u, 0u};
        }
        return;
    }
    if (tid == 0) {
        int st = 0;
        for (int bb = 0; bb < e; ++bb) st += s_hist[bb];
        s_start = st;
    }
    if (!SPEC) load_b();

    __syncthreads();
    const int start = s_start;

    // 3. 16-row sub-tiles of this expert's assignments. The rows of sub-tile m0 + 16 are
    // requested right after sub-tile m0's MFMAs are issued, so their latency overlaps its
    // reduction and epilogue (the MFMAs have read the registers the new rows land in).
    u32x4 a[S];
    auto load_a = [&](int m0) {
        const int j = m0 + r;
        if (j < count) {
            const bf16_t* a_src = GATEUP ? p.A + (int64_t)(s_rows[j] / p.top_k) * p.K + kbase
                                         : p.A + (int64_t)(start + j) * p.K + kbase;
            const u32x4* src = reinterpret_cast<const u32x4*>(a_src);
#pragma unroll
            for (int s = 0; s < S; ++s) a[s] = src[4 * s];
        } else {
#pragma unroll
            for (int s = 0; s < S; ++s) a[s] = u32x4{0u, 0u, 0u, 0u};
        }
    };
    load_a(0);
    for (int m0 = 0; m0 < count; m0 += 16) {
        f32x4 acc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[s]),
                                                                  as_bf16x8(b[nb][s]), acc[nb],
                                                                  0, 0, 0);
        if (m0 + 16 < count) load_a(m0 + 16);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) red[wave][wgrp * NB + nb][lane] = acc[nb];
        __syncthreads();
        // thread (l, i, g) finalises row (l/16)*4 + i, column l%16 of the blocks of group g
        const int l = tid & 63, i = (tid >> 6) & 3;
        const int row = (l >> 4) * 4 + i, col = l & 15;
        if (m0 + row < count) {
            float v[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int bb = wgrp * NB + nb;
                v[nb] = ((red[0][bb][l][i] + red[1][bb][l][i]) + red[2][bb][l][i]) +
                        red[3][bb][l][i];
            }
            if (GATEUP) {
                p.C[(int64_t)(start + m0 + row) * p.N + (n_tile * WN + wgrp) * 16 + col] =
                    f32_to_bf16(swiglu_bf16(v[0], v[1]));
            } else {
                const int flat = s_rows[m0 + row];
                const float w = p.topk_w[flat];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    p.C[(int64_t)flat * p.N + n_tile * OUTC + (wgrp * NB + nb) * 16 + col] =
                        f32_to_bf16(v[nb] * w);
            }
        }
        __syncthreads();
    }
}

template <int S, int NB, bool GATEUP, bool PACKED, int WN = 1>
void launch_e(const ExpertArgs& g, hipStream_t stream) {
    const int experts = g.E + (GATEUP ? 0 : 1);
    if (2 * g.numel < g.E) {
        // few assignments: one workgroup column per non-empty bucket (at most numel of them)
        const int cols = (int)(g.numel < experts ? g.numel : experts);
        hipLaunchKernelGGL((moe_expert_kernel<S, NB, WN, GATEUP, PACKED, 2>),
                           dim3(cols * g.n_tiles), dim3(256 * WN), 0, stream, g);
    } else if (g.numel >= 2ll * g.E) {
        // speculative weight loads once an expert is expected to see >= 2 assignments
        hipLaunchKernelGGL((moe_expert_kernel<S, NB, WN, GATEUP, PACKED, 1>),
                           dim3(experts * g.n_tiles), dim3(256 * WN), 0, stream, g);
    } else {
        hipLaunchKernelGGL((moe_expert_kernel<S, NB, WN, GATEUP, PACKED, 0>),
                           dim3(experts * g.n_tiles), dim3(256 * WN), 0, stream, g);
    }
}

// gate_up with WN wavefront groups (16 activation columns each) per workgroup.
template <bool PACKED, int WN>
bool gate_up_wn(ExpertArgs g, hipStream_t stream) {
    g.n_tiles = g.N / (16 * WN);
    switch (g.K / 128) {
        case 2: launch_e<2, 2, true, PACKED, WN>(g, stream); return true;
        case 4: launch_e<4, 2, true, PACKED, WN>(g, stream); return true;
        case 6: launch_e<6, 2, true, PACKED, WN>(g, stream); return true;
        case 8: launch_e<8, 2, true, PACKED, WN>(g, stream); return true;
        case 12: launch_e<12, 2, true, PACKED, WN>(g, stream); return true;
        case 16: launch_e<16, 2, true, PACKED, WN>(g, stream); return true;
        default: return false;
    }
}

template <bool PACKED>
bool gate_up_e(const ExpertArgs& g, hipStream_t stream) {
    // one wavefront group: two (8 waves at ~210 VGPRs, one workgroup per CU) measured slower
    // at every batch size although they halve the gathered x reads
    return gate_up_wn<PACKED, 1>(g, stream);
}

template <bool PACKED>
bool down_e(ExpertArgs g, hipStream_t stream) {
    const int S = g.K / 128;
    if (S <= 8 && g.N % 64 == 0) {
        g.n_tiles = g.N / 64;
        switch (S) {
            case 2: launch_e<2, 4, false, PACKED>(g, stream); return true;
            case 4: launch_e<4, 4, false, PACKED>(g, stream); return true;
            case 6: launch_e<6, 4, false, PACKED>(g, stream); return true;
            case 8: launch_e<8, 4, false, PACKED>(g, stream); return true;
            default: return false;
        }
    }
    if (g.N % 32 != 0) return false;
    g.n_tiles = g.N / 32;
    switch (S) {
        case 12: launch_e<12, 2, false, PACKED>(g, stream); return true;
        case 16: launch_e<16, 2, false, PACKED>(g, stream); return true;
        default: return false;
    }
}

}  // namespace

static bool has_s(int K) {  // K/128 values with an instantiation
    if (K % 128 != 0) return false;
    const int S = K / 128;
    return S == 2 || S == 4 || S == 6 || S == 8 || S == 12 || S == 16;
}

bool expert_path_supported(int64_t numel, int H, int I, int E) {
    return numel <= kExpertMaxRows && E + 1 <= kMaxBucketsE && has_s(H) && has_s(I) &&
           I % 16 == 0 && H % 128 == 0;
}

bool launch_expert_gate_up(ExpertArgs g, bool packed, hipStream_t stream) {
    if (g.N % 16 != 0 || g.K % 128 != 0) return false;
    return packed ? gate_up_e<true>(g, stream) : gate_up_e<false>(g, stream);
}

bool launch_expert_down(ExpertArgs g, bool packed, hipStream_t stream) {
    if (g.K % 128 != 0) return false;
    return packed ? down_e<true>(g, stream) : down_e<false>(g, stream);
}

}  // namespace tsm
