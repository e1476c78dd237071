// fp32 experts: fused_moe for fp32 activations and weights.
//
// Reference: fused_moe allocates its intermediates in x.dtype (tinykernels.py:1784-1791), so an
// fp32 layer (the tiny qwen3_moe configuration) computes x @ w13[e]^T, silu(gate) * up and
// (act @ w2[e]^T) * routing weight in fp32 and sums each token's k rows in fp32
// (tinykernels.py:1796); moe_reference (serve.py:933-996) does the same per expert.
//
// The matrix-core path is bf16; this one is fp32 throughout on the vector ALUs: 16 expert-sorted
// rows (the align step's 16-row tiles) x 64 output columns per workgroup, each of the 256 lanes
// owning one row and 4 columns (gate_up: 4 gate and the 4 matching up columns), with operand
// tiles of 32 k staged through LDS. Rows of the remote bucket (expert -1) produce zero rows in
// the down stage, as in the bf16 kernels.
#include <algorithm>
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

constexpr int kRows = 16;   // tile height (the align step's block_m)
constexpr int kCols = 64;   // output columns per workgroup
constexpr int kKC = 32;     // k per LDS stage

template <bool GATEUP>
__global__ __launch_bounds__(256) void moe_f32_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
    const float* __restrict__ topk_w, const int32_t* __restrict__ sorted_ids,
    const int32_t* __restrict__ expert_ids, const int32_t* __restrict__ total, int64_t numel,
    int top_k, int N, int K) {
    constexpr int NB = GATEUP ? 2 * kCols : kCols;   // B rows staged per k stage
    __shared__ float sA[kRows][kKC + 1];
    __shared__ float sB[NB][kKC + 1];
    const int m_tile = blockIdx.x;
    const int64_t m0 = (int64_t)m_tile * kRows;
    if (m0 >= total[0]) return;
    const int e = expert_ids[m_tile];
    const int n0 = blockIdx.y * kCols;
    const int tid = threadIdx.x, r = tid / 16, cg = tid % 16;
    const int flat_r = sorted_ids[m0 + r];
    const bool valid_r = flat_r < numel;

    if (e < 0) {  // assignments owned by another GPU: zero rows in the down stage
        if (!GATEUP && valid_r) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int n = n0 + cg * 4 + c;
                if (n < N) C[(int64_t)flat_r * N + n] = 0.0f;
            }
        }
        return;
    }
    const float* Be = B + (int64_t)e * (GATEUP ? 2 : 1) * N * K;
    float acc[4] = {0.f, 0.f, 0.f, 0.f}, up[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K; k0 += kKC) {
        // A: 16 rows x 32 k (gate_up: gathered token rows; down: the tile's own rows)
        for (int idx = tid; idx < kRows * kKC; idx += 256) {
            const int rr = idx / kKC, kk = idx % kKC;
            const int flat = sorted_ids[m0 + rr];
            float v = 0.0f;
            if (flat < numel && k0 + kk < K) {
                const int64_t row = GATEUP ? flat / top_k : m0 + rr;
                v = A[row * K + k0 + kk];
            }
            sA[rr][kk] = v;
        }
        // B: the workgroup's weight rows (gate_up: gate rows n0.., then up rows N + n0..)
        for (int idx = tid; idx < NB * kKC; idx += 256) {
            const int rr = idx / kKC, kk = idx % kKC;
            const int n = n0 + (GATEUP ? rr % kCols : rr);
            float v = 0.0f;
            if (n < N && k0 + kk < K) {
                const int64_t brow = GATEUP && rr >= kCols ? N + n : n;
                v = Be[brow * K + k0 + kk];
            }
            sB[rr][kk] = v;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < kKC; ++kk) {
            const float a = sA[r][kk];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                acc[c] = __builtin_fmaf(a, sB[cg * 4 + c][kk], acc[c]);
                if (GATEUP) up[c] = __builtin_fmaf(a, sB[kCols + cg * 4 + c][kk], up[c]);
            }
        }
        __syncthreads();
    }
    if (!valid_r) return;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int n = n0 + cg * 4 + c;
        if (n >= N) continue;
        if (GATEUP) {
            const float g = acc[c];
            C[(m0 + r) * N + n] = g / (1.0f + expf(-g)) * up[c];   // silu(gate) * up
        } else {
            C[(int64_t)flat_r * N + n] = acc[c] * topk_w[flat_r];
        }
    }
}

__global__ __launch_bounds__(256) void combine_f32_kernel(const float* __restrict__ rows,
                                                          float* __restrict__ out, int64_t T,
                                                          int H, int k) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= T * H) return;
    const int64_t t = idx / H, c = idx % H;
    float acc = 0.0f;
    for (int s = 0; s < k; ++s) acc += rows[(t * k + s) * H + c];   // slot order
    out[idx] = acc;
}

struct LayoutF32 {
    size_t sorted, expert_ids, total, hist, act, rows, bytes;
};

LayoutF32 layout_f32(int64_t T, int H, int I, int E, int top_k) {
    const int64_t numel = T * top_k;
    const int64_t mp = max_padded_rows(numel, E, kRows);
    LayoutF32 L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = align_up(off + bytes, 256);
        return at;
    };
    L.sorted = take(sizeof(int32_t) * mp);
    L.expert_ids = take(sizeof(int32_t) * (mp / kRows));
    L.total = take(sizeof(int32_t));
    L.hist = take(align_workspace_bytes(numel, E));
    L.act = take(sizeof(float) * mp * I);
    L.rows = take(sizeof(float) * numel * H);
    L.bytes = off;
    return L;
}

}  // namespace
}  // namespace tsm

using namespace tsm;

extern "C" size_t tsm_fused_moe_f32_workspace_size(int64_t T, int H, int I, int E, int top_k) {
    if (T < 0 || H <= 0 || I <= 0 || E <= 0 || top_k <= 0) return 0;
    return layout_f32(T, H, I, E, top_k).bytes;
}

extern "C" int tsm_fused_moe_f32(const float* x, const float* w13, const float* w2,
                                 const float* topk_w, const int32_t* topk_ids, int64_t T, int H,
                                 int I, int E, int top_k, int sum_topk, float* out, void* ws,
                                 size_t ws_bytes, hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(T >= 0 && T < (1ll << 24), TSM_E_ARG, "T out of range (%lld)", (long long)T);
    TSM_REQUIRE(H >= 1 && I >= 1 && H <= (1 << 20) && I <= (1 << 20), TSM_E_SHAPE,
                "sizes out of range (H=%d I=%d)", H, I);
    TSM_REQUIRE(top_k >= 1 && top_k <= 64, TSM_E_ARG, "top_k must be in [1, 64] (got %d)", top_k);
    int rc = check_align_args(T * top_k, E, kRows);
    if (rc) return rc;
    if (T == 0) return TSM_OK;
    TSM_REQUIRE(x && w13 && w2 && topk_w && topk_ids && out, TSM_E_ARG, "null pointer argument");
    TSM_REQUIRE(tsm_aligned(4, {x, w13, w2, topk_w, topk_ids, out}), TSM_E_ARG,
                "fp32 tensors must be 4-byte aligned");
    const LayoutF32 L = layout_f32(T, H, I, E, top_k);
    TSM_REQUIRE(ws && ws_bytes >= L.bytes && ((uintptr_t)ws & 255) == 0, TSM_E_WORKSPACE,
                "workspace must be 256-byte aligned and >= %zu bytes (got %zu)", L.bytes,
                ws_bytes);
    char* w = (char*)ws;
    const int64_t numel = T * top_k;
    int32_t* sorted = reinterpret_cast<int32_t*>(w + L.sorted);
    int32_t* eids = reinterpret_cast<int32_t*>(w + L.expert_ids);
    int32_t* total = reinterpret_cast<int32_t*>(w + L.total);
    float* act = reinterpret_cast<float*>(w + L.act);
    float* rows = sum_topk ? reinterpret_cast<float*>(w + L.rows) : out;
    rc = launch_status(launch_align(topk_ids, numel, E, kRows, sorted, eids, total, w + L.hist,
                                    stream),
                       "fused_moe_f32 align kernels");
    if (rc) return rc;
    const unsigned m_tiles = (unsigned)active_tile_bound(numel, E, kRows);
    hipLaunchKernelGGL(moe_f32_kernel<true>, dim3(m_tiles, (unsigned)((I + kCols - 1) / kCols)),
                       dim3(256), 0, stream, x, w13, act, (const float*)nullptr, sorted, eids,
                       total, numel, top_k, I, H);
    hipLaunchKernelGGL(moe_f32_kernel<false>, dim3(m_tiles, (unsigned)((H + kCols - 1) / kCols)),
                       dim3(256), 0, stream, (const float*)act, w2, rows, topk_w, sorted, eids,
                       total, numel, 1, H, I);
    if (sum_topk)
        hipLaunchKernelGGL(combine_f32_kernel, dim3((unsigned)((T * H + 255) / 256)), dim3(256),
                           0, stream, (const float*)rows, out, T, H, top_k);
    return check_launch("fused_moe_f32 kernels");
}
