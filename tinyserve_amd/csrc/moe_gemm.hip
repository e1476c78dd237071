// Grouped expert GEMMs on expert-sorted rows, the SwiGLU activation, the fixed-order top-k
// combine, and the fused_moe / whole-layer entry points.
//
// Reference: fused_moe (tinykernels.py:1767-1796) -> _moe_gemm / _fused_moe_kernel
// (tinykernels.py:1589-1765) twice with silu_and_mul (tinykernels.py:280-307) in between and a
// torch k-sum at the end; numerics of each row follow the reference: gate/up outputs are rounded
// to bf16, silu(gate) is rounded to bf16 before the multiply by up, the down output is scaled by
// the fp32 routing weight and rounded to bf16; the k rows of a token are then summed in fp32.
//
// Differences in structure (not in results): the activation is computed in the epilogue of the
// gate_up GEMM (no [T*k, 2I] intermediate), the activation rows are stored in the expert-sorted
// order so the down GEMM reads contiguous rows, and the k-sum is a fixed-order pass (slot 0..k-1)
// rather than a reduction of unspecified order.
#include <algorithm>
#include <atomic>
#include <mutex>
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

constexpr int BK = 64;        // K elements per main-loop step
constexpr int LDK = BK + 8;   // LDS row stride in bf16 elements (144 bytes: 16-byte aligned rows)


// Workgroup tile BM x BN of C (for gate_up, BN counts B rows: BN/2 gate rows + the matching BN/2
// up rows, so BN/2 activation columns), 4 wavefronts in a WM x WN grid, 16x16x32 bf16 MFMA,
// A and B staged through double-buffered LDS with a register prefetch of the next K step.
template <int BM, int BN, int WM, int WN, bool GATEUP, bool PACKED>
__global__ __launch_bounds__(256) void moe_gemm_kernel(GemmArgs p) {
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int A_CHUNKS = BM * (BK / 8), B_CHUNKS = BN * (BK / 8);
    constexpr int CA = (A_CHUNKS + 255) / 256, CB = B_CHUNKS / 256;
    static_assert(WM * WN == 4, "4 wavefronts");
    static_assert(FM >= 1 && FN >= 1 && B_CHUNKS % 256 == 0, "tile shape");
    static_assert(!GATEUP || FN % 2 == 0, "gate_up wave tile needs gate and up blocks");
    __shared__ __attribute__((aligned(16))) bf16_t sA[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) bf16_t sB[2][BN * LDK];

    // XCD-aware tile order: workgroup i runs on XCD i % 8; give each XCD a contiguous range of
    // logical tiles so that tiles sharing an expert's weight panel meet in the same L2.
    const int G = p.m_tiles * p.n_tiles;
    const int pid = blockIdx.x;
    const int xcd = pid & 7, q = G >> 3, r = G & 7;
    const int logical = xcd * q + min(xcd, r) + (pid >> 3);
    const int m_tile = logical % p.m_tiles, n_tile = logical / p.m_tiles;
    const int m0 = m_tile * BM;
    if (m0 >= p.total[0]) return;
    const int expert = p.expert_ids[m_tile];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    if (expert < 0) {  // assignments owned by another GPU: zero rows, no GEMM
        if (!GATEUP) {
            for (int idx = tid; idx < BM * (BN / 8); idx += 256) {
                const int row = idx / (BN / 8), cc = idx % (BN / 8);
                const int flat = p.sorted_ids[m0 + row];
                if (flat < p.numel)
                    *reinterpret_cast<u32x4*>(p.C + (int64_t)flat * p.N + n_tile * BN + cc * 8) =
                        u32x4{0u, 0u, 0u, 0u};
            }
        }
        return;
    }

    const bf16_t* a_src[CA];
#pragma unroll
    for (int c = 0; c < CA; ++c) {
        const int idx = tid + c * 256;
        const bf16_t* s = nullptr;
        if (idx < A_CHUNKS) {
            const int row = idx / (BK / 8), kc = idx % (BK / 8);
            if (GATEUP) {
                const int flat = p.sorted_ids[m0 + row];
                if (flat < p.numel) s = p.A + (int64_t)(flat / p.top_k) * p.K + kc * 8;
            } else {
                s = p.A + (int64_t)(m0 + row) * p.K + kc * 8;
            }
        }
        a_src[c] = s;
    }
    const bf16_t* Be = p.B + (int64_t)expert * (GATEUP ? 2 : 1) * p.N * p.K;
    const bf16_t* b_src[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
        const int idx = tid + c * 256;
        const int row = idx / (BK / 8), kc = idx % (BK / 8);
        int brow;
        if (GATEUP)
            brow = row < BN / 2 ? n_tile * (BN / 2) + row : p.N + n_tile * (BN / 2) + row - BN / 2;
        else
            brow = n_tile * BN + row;
        if (PACKED) {  // MFMA-tiled layout (moe_pack.hip); w13 blocks interleave gate/up
            const int blk = GATEUP ? (brow < p.N ? 2 * (brow >> 4) : 2 * ((brow - p.N) >> 4) + 1)
                                   : (brow >> 4);
            b_src[c] = Be + (((int64_t)blk * (p.K / 32) + (kc >> 2)) * 64 + (brow & 15) +
                             16 * (kc & 3)) * 8;
        } else {
            b_src[c] = Be + (int64_t)brow * p.K + kc * 8;
        }
    }
    constexpr int kBStep = PACKED ? (BK / 32) * 512 : BK;  // elements per K step

    u32x4 ra[CA], rb[CB];
    auto gload = [&](int kt) {
#pragma unroll
        for (int c = 0; c < CA; ++c)
            ra[c] = a_src[c] ? *reinterpret_cast<const u32x4*>(a_src[c] + kt * BK)
                             : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int c = 0; c < CB; ++c)
            rb[c] = *reinterpret_cast<const u32x4*>(b_src[c] + kt * kBStep);
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int c = 0; c < CA; ++c) {
            const int idx = tid + c * 256;
            if (idx < A_CHUNKS) {
                const int row = idx / (BK / 8), kc = idx % (BK / 8);
                *reinterpret_cast<u32x4*>(&sA[buf][row * LDK + kc * 8]) = ra[c];
            }
        }
#pragma unroll
        for (int c = 0; c < CB; ++c) {
            const int idx = tid + c * 256;
            const int row = idx / (BK / 8), kc = idx % (BK / 8);
            *reinterpret_cast<u32x4*>(&sB[buf][row * LDK + kc * 8]) = rb[c];
        }
    };

    const int wm = wave / WN, wn = wave % WN;
    constexpr int OW = WTN / 2;  // gate_up: activation columns per wavefront
    auto brow_of = [&](int g) {
        if (GATEUP)
            return g < FN / 2 ? wn * OW + g * 16 : BN / 2 + wn * OW + (g - FN / 2) * 16;
        return wn * WTN + g * 16;
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int f = 0; f < FM; ++f)
#pragma unroll
        for (int g = 0; g < FN; ++g) acc[f][g] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int KT = p.K / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int koff = ks * 32 + (lane >> 4) * 8;
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int f = 0; f < FM; ++f) {
                const int row = wm * WTM + f * 16 + (lane & 15);
                af[f] = as_bf16x8(*reinterpret_cast<const u32x4*>(&sA[buf][row * LDK + koff]));
            }
#pragma unroll
            for (int g = 0; g < FN; ++g) {
                const int row = brow_of(g) + (lane & 15);
                bfr[g] = as_bf16x8(*reinterpret_cast<const u32x4*>(&sB[buf][row * LDK + koff]));
            }
#pragma unroll
            for (int f = 0; f < FM; ++f)
#pragma unroll
                for (int g = 0; g < FN; ++g)
                    acc[f][g] =
                        __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[f], bfr[g], acc[f][g], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue. Accumulator element i of block (f, g) is row (lane/16)*4 + i, column lane%16.
#pragma unroll
    for (int f = 0; f < FM; ++f) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int grow = m0 + wm * WTM + f * 16 + (lane >> 4) * 4 + i;
            if (GATEUP) {
#pragma unroll
                for (int g = 0; g < FN / 2; ++g) {
                    const int col = n_tile * (BN / 2) + wn * OW + g * 16 + (lane & 15);
                    p.C[(int64_t)grow * p.N + col] =
                        f32_to_bf16(swiglu_bf16(acc[f][g][i], acc[f][g + FN / 2][i]));
                }
            } else {
                const int flat = p.sorted_ids[grow];
                if (flat < p.numel) {
                    const float w = p.topk_w[flat];
#pragma unroll
                    for (int g = 0; g < FN; ++g) {
                        const int col = n_tile * BN + wn * WTN + g * 16 + (lane & 15);
                        p.C[(int64_t)flat * p.N + col] = f32_to_bf16(acc[f][g][i] * w);
                    }
                }
            }
        }
    }
}

// out[t, :] = bf16(sum over s = 0..k-1 of rows[t*k + s, :]) with fp32 accumulation in slot order.
// STREAM: rows larger than the L2s are read and the output written with non-temporal accesses;
// smaller rows were just written by the down GEMM and are read from L2.
template <bool STREAM>
__global__ __launch_bounds__(256) void combine_kernel(const bf16_t* __restrict__ rows,
                                                      bf16_t* __restrict__ out, int64_t T, int H,
                                                      int k) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int cpr = H / 8;
    const int64_t t = idx / cpr;
    const int c = (int)(idx % cpr);
    if (t >= T) return;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < k; ++s) {
        const u32x4* src = reinterpret_cast<const u32x4*>(rows + ((t * k + s) * H + c * 8));
        const u32x4 v = STREAM ? __builtin_nontemporal_load(src) : *src;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[2 * j] += lo_bf16(v[j]);
            acc[2 * j + 1] += hi_bf16(v[j]);
        }
    }
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = pack_bf16(acc[2 * j], acc[2 * j + 1]);
    u32x4* dst = reinterpret_cast<u32x4*>(out + (t * H + c * 8));
    if (STREAM) __builtin_nontemporal_store(o, dst);
    else *dst = o;
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const bf16_t* __restrict__ gate,
                                                       int64_t gs, const bf16_t* __restrict__ up,
                                                       int64_t us, bf16_t* __restrict__ out,
                                                       int64_t os, int64_t N) {
    const int64_t row = blockIdx.y;
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < N;
         c += (int64_t)gridDim.x * 256) {
        out[row * os + c] = f32_to_bf16(
            swiglu_bf16(bf16_to_f32(gate[row * gs + c]), bf16_to_f32(up[row * us + c])));
    }
}

// ---- kernel table --------------------------------------------------------------------------
// Tile height per batch size. block_m == 0: expert-major weight streaming (moe_expert.hip, no
// permutation step) up to numel = 12E (above that the align step plus 64-row pipelined tiles
// measured faster with packed weights: T=256 of the Qwen3-30B layer 233 vs 256 us for the GEMM
// stages; both layouts switch at the same size, so they keep giving the same bits): from 2E on
// with the weights requested before the id scan, below E/2 with one workgroup column per
// non-empty expert instead of per expert. Otherwise
// reference-layout weights use 64-row LDS tiles (the reference's BLOCK_M switch is at 4E,
// tinykernels.py:1779); packed weights use 64-row pipelined tiles up to 32E and 128-row above.
struct Plan {
    int block_m;
};

bool block_m_supported(int block_m, bool packed);

// Tile heights installed by autotuning (tsm_moe_set_block_m), per weight layout and per
// power-of-two bucket of the assignment count (bucket b holds numel in [2^b, 2^(b+1))); -1 = the
// static table. Read on every plan, written rarely: relaxed atomics.
constexpr int kBuckets = 40;
std::atomic<int> g_block_m_override[2][kBuckets];
std::once_flag g_override_init;

void init_overrides() {
    for (auto& layout : g_block_m_override)
        for (auto& b : layout) b.store(-1, std::memory_order_relaxed);
}

int numel_bucket(int64_t numel) {
    int b = 0;
    while (b + 1 < kBuckets && (int64_t(1) << (b + 1)) <= numel) ++b;
    return b;
}

Plan plan_for(int64_t T, int H, int I, int E, int top_k, bool packed) {
    const int64_t numel = T * top_k;
    std::call_once(g_override_init, init_overrides);
    if (numel >= 1) {
        const int o = g_block_m_override[packed][numel_bucket(numel)].load(std::memory_order_relaxed);
        // an installed height applies where its kernels take the shape
        if (o == 0 && expert_path_supported(numel, H, I, E)) return Plan{0};
        if (o > 0 && block_m_supported(o, packed) && (o < 128 || tile_kernels_take(H, I)) &&
            (o != 256 || tile256_takes_x(T, H)))
            return Plan{o};
    }
    if (numel >= 1 && numel <= 12ll * E && expert_path_supported(numel, H, I, E))
        return Plan{0};
    if (numel <= 4ll * E) return Plan{16};
    // 128-row tiles exist only as the pipelined tile kernels, which need their shapes
    if (!packed || numel <= 32ll * E || !tile_kernels_take(H, I)) return Plan{64};
    return Plan{128};
}

constexpr int kBN = 128;  // B rows per workgroup tile (both variants)

struct Layout {
    size_t sorted, expert_ids, total, hist, act, rows, topk_w, topk_ids, logits, bytes;
};

Layout layout_for(int64_t T, int H, int I, int E, int top_k, bool with_route) {
    // Every buffer sized for whichever tile height (reference or packed layout) needs more: the
    // padded row count grows with block_m, the tile count shrinks with it.
    const int64_t numel = T * top_k;
    int64_t mp = 0, tiles = 0;
    for (bool packed : {false, true}) {
        const int bm = plan_for(T, H, I, E, top_k, packed).block_m;
        if (bm == 0) {  // expert-major path: compact activations, no permutation buffers
            mp = std::max(mp, numel);
            continue;
        }
        const int64_t m = max_padded_rows(numel, E, bm);
        mp = std::max(mp, m);
        tiles = std::max(tiles, m / bm);
    }
    Layout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = align_up(off + bytes, 256);
        return at;
    };
    L.sorted = take(sizeof(int32_t) * mp);
    L.expert_ids = take(sizeof(int32_t) * tiles);
    L.total = take(sizeof(int32_t));
    L.hist = take(align_workspace_bytes(numel, E));
    L.act = take(sizeof(bf16_t) * mp * I);
    L.rows = take(sizeof(bf16_t) * numel * H);
    if (with_route) {
        L.topk_w = take(sizeof(float) * numel);
        L.topk_ids = take(sizeof(int32_t) * numel);
        L.logits = take(sizeof(float) * T * E);  // router logits, staged for the selection
    }
    L.bytes = off;
    return L;
}

int check_moe_shapes(int64_t T, int H, int I, int E, int top_k) {
    TSM_REQUIRE(T >= 0 && T < (1ll << 24), TSM_E_ARG, "T out of range (%lld)", (long long)T);
    TSM_REQUIRE(H >= 64 && H % kBN == 0, TSM_E_SHAPE, "H must be a positive multiple of %d (got %d)",
                kBN, H);
    TSM_REQUIRE(I >= 64 && I % (kBN / 2) == 0, TSM_E_SHAPE,
                "I must be a positive multiple of %d (got %d)", kBN / 2, I);
    TSM_REQUIRE(top_k >= 1 && top_k <= 64, TSM_E_ARG, "top_k must be in [1, 64] (got %d)", top_k);
    return check_align_args(T * top_k, E, 64);
}

GemmArgs gemm_args(const bf16_t* A, const bf16_t* B, bf16_t* C, const float* topk_w,
                   const int32_t* sorted, const int32_t* eids, const int32_t* total,
                   int64_t numel, int top_k, int N, int K, int E, int block_m, int n_tiles) {
    GemmArgs g{};
    g.A = A;
    g.B = B;
    g.C = C;
    g.topk_w = topk_w;
    g.sorted_ids = sorted;
    g.expert_ids = eids;
    g.total = total;
    g.numel = numel;
    g.top_k = top_k;
    g.N = N;
    g.K = K;
    g.m_tiles = (int)active_tile_bound(numel, E, block_m);
    g.n_tiles = n_tiles;
    return g;
}

bool block_m_supported(int block_m, bool packed) {
    if (block_m == 0) return false;  // the expert-major path has its own entry points
    // 128 and 256 rows: the pipelined tile kernels, packed weights only (256 is never chosen by
    // the static table; it is installed by autotuning where it measures faster)
    return block_m == 16 || block_m == 64 || (packed && (block_m == 128 || block_m == 256));
}

// gate_up GEMM + SwiGLU: act[max_padded, I] from x[T, H] and w13[E, 2I, H].
template <int BM, int WM, int WN, bool GATEUP>
void launch_lds(const GemmArgs& g, bool packed, hipStream_t stream) {
    const dim3 grid(g.m_tiles * g.n_tiles);
    if (packed)
        hipLaunchKernelGGL((moe_gemm_kernel<BM, kBN, WM, WN, GATEUP, true>), grid, dim3(256), 0,
                           stream, g);
    else
        hipLaunchKernelGGL((moe_gemm_kernel<BM, kBN, WM, WN, GATEUP, false>), grid, dim3(256), 0,
                           stream, g);
}

// false: no kernel for this tile height and shape (nothing launched). 128- and 256-row tiles have
// only the pipelined tile kernel; 16 and 64 fall back to the LDS kernel of their own height.
bool launch_gate_up(const bf16_t* x, const bf16_t* w13, const int32_t* sorted,
                    const int32_t* eids, const int32_t* total, int64_t numel, int top_k, int H,
                    int I, int E, int block_m, bool packed, bf16_t* act, hipStream_t stream) {
    GemmArgs g = gemm_args(x, w13, act, nullptr, sorted, eids, total, numel, top_k, I, H, E,
                           block_m, I / (kBN / 2));
    if (block_m == 16 && launch_stream_gate_up(g, packed, stream)) return true;
    if (packed && block_m >= 64 && launch_tile_gate_up(g, block_m, stream)) return true;
    if (block_m != 16 && block_m != 64) return false;
    if (block_m == 16)
        launch_lds<16, 1, 4, true>(g, packed, stream);
    else
        launch_lds<64, 2, 2, true>(g, packed, stream);
    return true;
}

// down GEMM * routing weight: rows[numel, H] from act[max_padded, I] and w2[E, H, I].
bool launch_down(const bf16_t* act, const bf16_t* w2, const float* topk_w, const int32_t* sorted,
                 const int32_t* eids, const int32_t* total, int64_t numel, int H, int I, int E,
                 int block_m, bool packed, bf16_t* rows, hipStream_t stream) {
    GemmArgs g = gemm_args(act, w2, rows, topk_w, sorted, eids, total, numel, 1, H, I, E,
                           block_m, H / kBN);
    if (block_m == 16 && launch_stream_down(g, packed, stream)) return true;
    if (packed && block_m >= 64 && launch_tile_down(g, block_m, stream)) return true;
    if (block_m != 16 && block_m != 64) return false;
    if (block_m == 16)
        launch_lds<16, 1, 4, false>(g, packed, stream);
    else
        launch_lds<64, 2, 2, false>(g, packed, stream);
    return true;
}

void launch_combine(const bf16_t* rows, int64_t T, int H, int top_k, bf16_t* out,
                    hipStream_t stream) {
    const int64_t threads = T * (H / 8);
    const dim3 grid((unsigned)((threads + 255) / 256));
    if ((int64_t)T * top_k * H * 2 > (32ll << 20))  // beyond the combined L2 of the 8 XCDs
        hipLaunchKernelGGL(combine_kernel<true>, grid, dim3(256), 0, stream, rows, out, T, H,
                           top_k);
    else
        hipLaunchKernelGGL(combine_kernel<false>, grid, dim3(256), 0, stream, rows, out, T, H,
                           top_k);
}

ExpertArgs expert_args(const bf16_t* A, const bf16_t* B, bf16_t* C, const float* topk_w,
                       const int32_t* ids, int64_t numel, int top_k, int N, int K, int E) {
    ExpertArgs g{};
    g.A = A;
    g.B = B;
    g.C = C;
    g.topk_w = topk_w;
    g.ids = ids;
    g.numel = numel;
    g.top_k = top_k;
    g.N = N;
    g.K = K;
    g.E = E;
    return g;
}

bool launch_expert_stages(const bf16_t* x, const bf16_t* w13, const bf16_t* w2,
                          const float* topk_w, const int32_t* ids, int64_t numel, int top_k,
                          int H, int I, int E, bool packed, bf16_t* act, bf16_t* rows,
                          hipStream_t stream) {
    if (!launch_expert_gate_up(expert_args(x, w13, act, nullptr, ids, numel, top_k, I, H, E),
                               packed, stream))
        return false;
    return launch_expert_down(expert_args(act, w2, rows, topk_w, ids, numel, 1, H, I, E), packed,
                              stream);
}

// Everything after routing: align, gate_up + SwiGLU, down * weight, k-sum.
int run_experts(const void* x, const void* w13, const void* w2, const float* topk_w,
                const int32_t* topk_ids, int64_t T, int H, int I, int E, int top_k, int sum_topk,
                bool packed, void* out, char* ws, const Layout& L, hipStream_t stream) {
    int rc = TSM_OK;
    const Plan pl = plan_for(T, H, I, E, top_k, packed);
    const int64_t numel = T * top_k;
    bf16_t* rows = sum_topk ? reinterpret_cast<bf16_t*>(ws + L.rows) : (bf16_t*)out;
    if (pl.block_m == 0) {
        TSM_REQUIRE(L.rows - L.act >= sizeof(bf16_t) * (size_t)(numel * I), TSM_E_WORKSPACE,
                    "internal: workspace layout does not fit the expert-major path");
        bf16_t* act = reinterpret_cast<bf16_t*>(ws + L.act);
        TSM_REQUIRE(launch_expert_stages((const bf16_t*)x, (const bf16_t*)w13,
                                         (const bf16_t*)w2, topk_w, topk_ids, numel, top_k, H,
                                         I, E, packed, act, rows, stream),
                    TSM_E_SHAPE, "internal: no expert-major kernel for H=%d I=%d", H, I);
        if (sum_topk) launch_combine(rows, T, H, top_k, (bf16_t*)out, stream);
        return check_launch("fused_moe kernels");
    }
    {   // the workspace regions must hold this plan's buffers (host-side guard, no launch if not)
        const int64_t mp = max_padded_rows(numel, E, pl.block_m);
        const bool fits = L.expert_ids - L.sorted >= sizeof(int32_t) * (size_t)mp &&
                          L.total - L.expert_ids >= sizeof(int32_t) * (size_t)(mp / pl.block_m) &&
                          L.rows - L.act >= sizeof(bf16_t) * (size_t)(mp * I);
        TSM_REQUIRE(fits, TSM_E_WORKSPACE, "internal: workspace layout does not fit block_m %d",
                    pl.block_m);
    }
    int32_t* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
    int32_t* eids = reinterpret_cast<int32_t*>(ws + L.expert_ids);
    int32_t* total = reinterpret_cast<int32_t*>(ws + L.total);
    bf16_t* act = reinterpret_cast<bf16_t*>(ws + L.act);

    rc = launch_status(
        launch_align(topk_ids, numel, E, pl.block_m, sorted, eids, total, ws + L.hist, stream),
        "fused_moe align kernels");
    if (rc) return rc;
    TSM_REQUIRE(launch_gate_up((const bf16_t*)x, (const bf16_t*)w13, sorted, eids, total, numel,
                               top_k, H, I, E, pl.block_m, packed, act, stream) &&
                    launch_down(act, (const bf16_t*)w2, topk_w, sorted, eids, total, numel, H, I,
                                E, pl.block_m, packed, rows, stream),
                TSM_E_SHAPE, "internal: no %d-row kernel for H=%d I=%d", pl.block_m, H, I);
    if (sum_topk) launch_combine(rows, T, H, top_k, (bf16_t*)out, stream);
    return check_launch("fused_moe kernels");
}

}  // namespace
}  // namespace tsm

using namespace tsm;

extern "C" int tsm_moe_set_block_m(int64_t numel_lo, int64_t numel_hi, int weight_layout,
                                   int block_m) {
    clear_error();
    TSM_REQUIRE(numel_lo >= 1 && numel_hi >= numel_lo, TSM_E_ARG,
                "need 1 <= numel_lo <= numel_hi (got %lld, %lld)", (long long)numel_lo,
                (long long)numel_hi);
    TSM_REQUIRE(weight_layout == TSM_LAYOUT_REFERENCE || weight_layout == TSM_LAYOUT_PACKED,
                TSM_E_ARG, "unknown weight layout %d", weight_layout);
    TSM_REQUIRE(block_m == -1 || block_m == 0 || block_m_supported(block_m, weight_layout != 0),
                TSM_E_SHAPE, "block_m %d has no kernel for this weight layout", block_m);
    std::call_once(g_override_init, init_overrides);
    for (int b = numel_bucket(numel_lo); b <= numel_bucket(numel_hi); ++b)
        g_block_m_override[weight_layout != 0][b].store(block_m, std::memory_order_relaxed);
    return TSM_OK;
}

extern "C" int tsm_moe_block_m(int64_t T, int H, int I, int E, int top_k, int weight_layout) {
    (void)H;
    (void)I;
    return plan_for(T, H, I, E, top_k, weight_layout != 0).block_m;
}

extern "C" int tsm_silu_and_mul(const void* gate, int64_t gate_stride, const void* up,
                                int64_t up_stride, void* out, int64_t out_stride, int64_t rows,
                                int64_t N, hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(rows >= 0 && N >= 0 && rows < 65536ll * 1024, TSM_E_ARG, "bad sizes");
    if (rows == 0 || N == 0) return TSM_OK;
    TSM_REQUIRE(gate && up && out, TSM_E_ARG, "null pointer argument");
    const unsigned gx = (unsigned)std::min<int64_t>((N + 255) / 256, 64);
    // gridDim.y is limited to 65535: process rows in bands
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
        const int64_t nr = std::min<int64_t>(65535, rows - r0);
        hipLaunchKernelGGL(silu_mul_kernel, dim3(gx, (unsigned)nr), dim3(256), 0, stream,
                           (const bf16_t*)gate + r0 * gate_stride, gate_stride,
                           (const bf16_t*)up + r0 * up_stride, up_stride,
                           (bf16_t*)out + r0 * out_stride, out_stride, N);
    }
    return check_launch("silu_mul_kernel");
}

extern "C" size_t tsm_fused_moe_workspace_size(int64_t T, int H, int I, int E, int top_k) {
    if (T < 0 || H <= 0 || I <= 0 || E <= 0 || top_k <= 0) return 0;
    return layout_for(T, H, I, E, top_k, false).bytes;
}

static int fused_moe_impl(const void* x, const void* w13, const void* w2, const float* topk_w,
                          const int32_t* topk_ids, int64_t T, int H, int I, int E, int top_k,
                          int sum_topk, bool packed, void* out, void* ws, size_t ws_bytes,
                          hipStream_t stream) {
    clear_error();
    int rc = check_moe_shapes(T, H, I, E, top_k);
    if (rc) return rc;
    if (T == 0) return TSM_OK;
    TSM_REQUIRE(x && w13 && w2 && topk_w && topk_ids && out, TSM_E_ARG, "null pointer argument");
    TSM_REQUIRE(tsm_aligned(16, {x, w13, w2, out}), TSM_E_ARG,
                "x, weights and out must be 16-byte aligned");
    const Layout L = layout_for(T, H, I, E, top_k, false);
    TSM_REQUIRE(ws && ws_bytes >= L.bytes && ((uintptr_t)ws & 255) == 0, TSM_E_WORKSPACE,
                "workspace must be 256-byte aligned and >= %zu bytes (got %zu)", L.bytes,
                ws_bytes);
    return run_experts(x, w13, w2, topk_w, topk_ids, T, H, I, E, top_k, sum_topk, packed, out,
                       (char*)ws, L, stream);
}

extern "C" int tsm_fused_moe(const void* x, const void* w13, const void* w2, const float* topk_w,
                             const int32_t* topk_ids, int64_t T, int H, int I, int E, int top_k,
                             int sum_topk, void* out, void* ws, size_t ws_bytes,
                             hipStream_t stream) {
    return fused_moe_impl(x, w13, w2, topk_w, topk_ids, T, H, I, E, top_k, sum_topk, false, out,
                          ws, ws_bytes, stream);
}

extern "C" int tsm_fused_moe_packed(const void* x, const void* w13p, const void* w2p,
                                    const float* topk_w, const int32_t* topk_ids, int64_t T, int H,
                                    int I, int E, int top_k, int sum_topk, void* out, void* ws,
                                    size_t ws_bytes, hipStream_t stream) {
    return fused_moe_impl(x, w13p, w2p, topk_w, topk_ids, T, H, I, E, top_k, sum_topk, true, out,
                          ws, ws_bytes, stream);
}

extern "C" size_t tsm_moe_forward_workspace_size(int64_t T, int H, int I, int E, int top_k) {
    if (T < 0 || H <= 0 || I <= 0 || E <= 0 || top_k <= 0) return 0;
    return layout_for(T, H, I, E, top_k, true).bytes;
}

static int moe_forward_impl(const void* x, const void* gate_w, const void* w13, const void* w2,
                            const int64_t* expert_map, const float* bias, int64_t T, int H, int I,
                            int E, int top_k, int renorm, int logits_bf16, int sum_topk,
                            bool packed, void* out, float* topk_w, int32_t* topk_ids, void* ws,
                            size_t ws_bytes, hipStream_t stream) {
    clear_error();
    int rc = check_moe_shapes(T, H, I, E, top_k);
    if (rc) return rc;
    if (T == 0) return TSM_OK;
    TSM_REQUIRE(x && gate_w && w13 && w2 && out, TSM_E_ARG, "null pointer argument");
    TSM_REQUIRE(tsm_aligned(16, {x, gate_w, w13, w2, out}), TSM_E_ARG,
                "x, weights and out must be 16-byte aligned");
    const Layout L = layout_for(T, H, I, E, top_k, true);
    TSM_REQUIRE(ws && ws_bytes >= L.bytes && ((uintptr_t)ws & 255) == 0, TSM_E_WORKSPACE,
                "workspace must be 256-byte aligned and >= %zu bytes (got %zu)", L.bytes,
                ws_bytes);
    char* w = (char*)ws;
    float* tw = topk_w ? topk_w : reinterpret_cast<float*>(w + L.topk_w);
    int32_t* ti = topk_ids ? topk_ids : reinterpret_cast<int32_t*>(w + L.topk_ids);
    rc = tsm_moe_router(x, gate_w, TSM_BF16, T, H, E, top_k, renorm, expert_map, bias,
                        logits_bf16, reinterpret_cast<float*>(w + L.logits), tw, ti, stream);
    if (rc) return rc;
    return run_experts(x, w13, w2, tw, ti, T, H, I, E, top_k, sum_topk, packed, out, w, L,
                       stream);
}

extern "C" int tsm_moe_forward(const void* x, const void* gate_w, const void* w13, const void* w2,
                               const int64_t* expert_map, const float* bias, int64_t T, int H,
                               int I, int E, int top_k, int renorm, int logits_bf16,
                               int sum_topk, void* out, float* topk_w, int32_t* topk_ids,
                               void* ws, size_t ws_bytes, hipStream_t stream) {
    return moe_forward_impl(x, gate_w, w13, w2, expert_map, bias, T, H, I, E, top_k, renorm,
                            logits_bf16, sum_topk, false, out, topk_w, topk_ids, ws, ws_bytes,
                            stream);
}

extern "C" int tsm_moe_forward_packed(const void* x, const void* gate_w, const void* w13p,
                                      const void* w2p, const int64_t* expert_map,
                                      const float* bias, int64_t T, int H, int I, int E,
                                      int top_k, int renorm, int logits_bf16, int sum_topk,
                                      void* out, float* topk_w, int32_t* topk_ids, void* ws,
                                      size_t ws_bytes, hipStream_t stream) {
    return moe_forward_impl(x, gate_w, w13p, w2p, expert_map, bias, T, H, I, E, top_k, renorm,
                            logits_bf16, sum_topk, true, out, topk_w, topk_ids, ws, ws_bytes,
                            stream);
}

extern "C" int tsm_moe_gemm_gate_up(const void* x, const void* w13, const int32_t* sorted_ids,
                                    const int32_t* expert_ids, const int32_t* total,
                                    int64_t numel, int top_k, int H, int I, int E, int block_m,
                                    int weight_layout, void* act, hipStream_t stream) {
    clear_error();
    int rc = check_moe_shapes(numel / (top_k > 0 ? top_k : 1), H, I, E, top_k);
    if (rc) return rc;
    TSM_REQUIRE(block_m_supported(block_m, weight_layout != 0), TSM_E_SHAPE,
                "block_m %d has no kernel for this weight layout", block_m);
    if (numel == 0) return TSM_OK;
    TSM_REQUIRE(x && w13 && sorted_ids && expert_ids && total && act, TSM_E_ARG,
                "null pointer argument");
    TSM_REQUIRE(launch_gate_up((const bf16_t*)x, (const bf16_t*)w13, sorted_ids, expert_ids,
                               total, numel, top_k, H, I, E, block_m, weight_layout != 0,
                               (bf16_t*)act, stream),
                TSM_E_SHAPE, "no %d-row gate_up kernel for H=%d I=%d", block_m, H, I);
    return check_launch("gate_up GEMM");
}

extern "C" int tsm_moe_gemm_down(const void* act, const void* w2, const float* topk_w,
                                 const int32_t* sorted_ids, const int32_t* expert_ids,
                                 const int32_t* total, int64_t numel, int H, int I, int E,
                                 int block_m, int weight_layout, void* rows,
                                 hipStream_t stream) {
    clear_error();
    int rc = check_moe_shapes(numel, H, I, E, 1);
    if (rc) return rc;
    TSM_REQUIRE(block_m_supported(block_m, weight_layout != 0), TSM_E_SHAPE,
                "block_m %d has no kernel for this weight layout", block_m);
    if (numel == 0) return TSM_OK;
    TSM_REQUIRE(act && w2 && topk_w && sorted_ids && expert_ids && total && rows, TSM_E_ARG,
                "null pointer argument");
    TSM_REQUIRE(launch_down((const bf16_t*)act, (const bf16_t*)w2, topk_w, sorted_ids,
                            expert_ids, total, numel, H, I, E, block_m, weight_layout != 0,
                            (bf16_t*)rows, stream),
                TSM_E_SHAPE, "no %d-row down kernel for H=%d I=%d", block_m, H, I);
    return check_launch("down GEMM");
}

extern "C" int tsm_moe_combine(const void* rows, int64_t T, int H, int top_k, void* out,
                               hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(T >= 0 && H > 0 && H % 8 == 0 && top_k >= 1, TSM_E_ARG, "bad combine sizes");
    if (T == 0) return TSM_OK;
    TSM_REQUIRE(rows && out, TSM_E_ARG, "null pointer argument");
    launch_combine((const bf16_t*)rows, T, H, top_k, (bf16_t*)out, stream);
    return check_launch("combine");
}

extern "C" int tsm_moe_expert_gate_up(const void* x, const void* w13, const int32_t* topk_ids,
                                      int64_t numel, int top_k, int H, int I, int E,
                                      int weight_layout, void* act, hipStream_t stream) {
    clear_error();
    int rc = check_moe_shapes(numel / (top_k > 0 ? top_k : 1), H, I, E, top_k);
    if (rc) return rc;
    TSM_REQUIRE(expert_path_supported(numel, H, I, E), TSM_E_SHAPE,
                "expert-major path unsupported for numel=%lld H=%d I=%d E=%d", (long long)numel,
                H, I, E);
    if (numel == 0) return TSM_OK;
    TSM_REQUIRE(x && w13 && topk_ids && act, TSM_E_ARG, "null pointer argument");
    TSM_REQUIRE(launch_expert_gate_up(expert_args((const bf16_t*)x, (const bf16_t*)w13,
                                                  (bf16_t*)act, nullptr, topk_ids, numel, top_k,
                                                  I, H, E),
                                      weight_layout != 0, stream),
                TSM_E_SHAPE, "no expert-major gate_up kernel for H=%d", H);
    return check_launch("expert gate_up");
}

extern "C" int tsm_moe_expert_down(const void* act, const void* w2, const float* topk_w,
                                   const int32_t* topk_ids, int64_t numel, int H, int I, int E,
                                   int weight_layout, void* rows, hipStream_t stream) {
    clear_error();
    int rc = check_moe_shapes(numel, H, I, E, 1);
    if (rc) return rc;
    TSM_REQUIRE(expert_path_supported(numel, H, I, E), TSM_E_SHAPE,
                "expert-major path unsupported for numel=%lld H=%d I=%d E=%d", (long long)numel,
                H, I, E);
    if (numel == 0) return TSM_OK;
    TSM_REQUIRE(act && w2 && topk_w && topk_ids && rows, TSM_E_ARG, "null pointer argument");
    TSM_REQUIRE(launch_expert_down(expert_args((const bf16_t*)act, (const bf16_t*)w2,
                                               (bf16_t*)rows, topk_w, topk_ids, numel, 1, H, I,
                                               E),
                                   weight_layout != 0, stream),
                TSM_E_SHAPE, "no expert-major down kernel for I=%d", I);
    return check_launch("expert down");
}
