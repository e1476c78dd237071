// Router kernels: fp32 softmax + top-k + renormalisation, optionally preceded by the router (gate)
// GEMM in the same launch, or (decode sizes, logits buffer given) in a launch of its own spread
// over expert slices.
//
// Reference behaviour: _moe_route_kernel / moe_route (tinykernels.py:1535-1583) and the torch router
// branch of SparseMoE.forward (serve.py:1089-1096). Selection is on p = exp(l - max l) with the
// lowest expert index winning ties, as the Triton kernel's first-index argmax does; weights are
// p / sum(selected p) (renormalise) or p / sum(all p).
//
// Every floating-point operation on this path has a fixed order and uses router_expf, so the
// logits, ids and weights are reproducible bit for bit by a sequential host program:
//   logit(t, e): lane j of a wavefront accumulates, with fmaf starting from +0, the products
//   x[t,h]*g[e,h] for h = c*512 + j*8 + i in increasing (c, i) order (h < H); the 64 lane partials are
//   then summed by the XOR butterfly of wave_sum_butterfly; bias[e] is added if given; the result is
//   rounded to bf16 if requested.
#include "common.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

constexpr int kMaxM = 8;          // experts per lane: E <= 512
constexpr int kRouterWaves = 16;  // wavefronts per router workgroup
// Largest batch routed by the split gate GEMM when a logits buffer is given
constexpr int64_t kSplitMaxT = 256;

// LDS words wave_select needs per wavefront: E <= 128 keys as (hi, lo) pairs, then up to 64
// selected (p, index) pairs.
constexpr int kSelectLds = 2 * 128 + 2 * 64;

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Softmax numerators, top-k and weights for one token whose logits lane j holds at
// v[q] = logit[j + 64 q]. Writes topk_w/topk_ids[0..k). All lanes of the wavefront must call it;
// `lds` is kSelectLds words of LDS owned by this wavefront.
// Order: largest p first, the lowest expert index among equal p. Every p is +0 or more, so with
// -inf for experts out of range its bits, sign-flipped, order like unsigned integers, and
// key(e) = (bits(p_e) ^ sign) << 32 | ~e is a total order in which the selection is the k
// largest keys. E <= 128: each key's rank (the number of larger keys) is counted directly,
// and rank r < k is slot r; independent compares instead of k dependent rounds. Larger E:
// k rounds of a wavefront argmax. Both give the same slots; sel_sum adds them in slot order.
__device__ __forceinline__ void wave_select(float (&v)[kMaxM], int E, int top_k, int renorm,
                                            const int64_t* __restrict__ expert_map,
                                            float* __restrict__ out_w,
                                            int32_t* __restrict__ out_ids, uint32_t* lds) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & (kWave - 1);
    const int nq = (E + 63) >> 6;  // slots in use (uniform): the loops below skip the rest
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int q = 0; q < kMaxM; ++q)
        if (q < nq && lane + 64 * q < E) m = fmaxf(m, v[q]);
    m = wave_max(m);

    float part = 0.0f;  // this lane's share of sum(p), ascending q
#pragma unroll
    for (int q = 0; q < kMaxM; ++q) {
        if (q < nq) {
            const bool in = lane + 64 * q < E;
            const float pe = router_expf(v[q] - m);
            v[q] = in ? pe : -__builtin_huge_valf();
            part = in ? part + pe : part;
        }
    }

    float sel_sum = 0.0f, my_v = 0.0f;
    int my_i = 0;
    if (nq <= 2) {
        uint64_t* keys = reinterpret_cast<uint64_t*>(lds);
        uint32_t* slots = lds + 2 * 128;
        uint64_t mine[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int e = lane + 64 * q;
            mine[q] = e < E ? ((uint64_t)(__float_as_uint(v[q]) ^ 0x80000000u) << 32) |
                                  (uint32_t)~e
                            : 0;
            if (q < nq) keys[e] = mine[q];
        }
        wave_lds_sync();
        int rank[2][2] = {{0, 0}, {0, 0}};  // two accumulators per key
#pragma unroll 4
        for (int e2 = 0; e2 < 64 * nq; e2 += 2) {
            const uint64_t k0 = keys[e2], k1 = keys[e2 + 1];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                if (q < nq) {
                    rank[q][0] += k0 > mine[q] ? 1 : 0;
                    rank[q][1] += k1 > mine[q] ? 1 : 0;
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int r = rank[q][0] + rank[q][1];
            if (q < nq && lane + 64 * q < E && r < top_k) {
                slots[2 * r] = __float_as_uint(v[q]);
                slots[2 * r + 1] = (uint32_t)(lane + 64 * q);
            }
        }
        wave_lds_sync();
        for (int s = 0; s < top_k; ++s) sel_sum = sel_sum + __uint_as_float(slots[2 * s]);
        if (lane < top_k) {
            my_v = __uint_as_float(slots[2 * lane]);
            my_i = (int)slots[2 * lane + 1];
        }
        wave_lds_sync();  // the caller may reuse the words
    } else {
        for (int s = 0; s < top_k; ++s) {
            float bv = -__builtin_huge_valf();
            int bi = 0x7fffffff;
#pragma unroll
            for (int q = 0; q < kMaxM; ++q)
                if (q < nq) {
                    const bool take = v[q] > bv;  // ascending q: the lowest index wins ties
                    bv = take ? v[q] : bv;
                    bi = take ? lane + 64 * q : bi;
                }
            wave_argmax(bv, bi);
            sel_sum = sel_sum + bv;
            my_v = lane == s ? bv : my_v;
            my_i = lane == s ? bi : my_i;
#pragma unroll
            for (int q = 0; q < kMaxM; ++q)
                if (q < nq) v[q] = bi == lane + 64 * q ? -__builtin_huge_valf() : v[q];
        }
    }
    float denom = renorm ? sel_sum : wave_sum_butterfly(part);
    if (lane < top_k) {
        out_w[lane] = my_v / denom;
        out_ids[lane] = expert_map ? (int32_t)expert_map[my_i] : (int32_t)my_i;
    }
}

template <typename TLog>
__device__ __forceinline__ float load_logit(const TLog* p, int64_t i);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_logit<bf16_t>(const bf16_t* p, int64_t i) {
    return bf16_to_f32(p[i]);
}

// One wavefront per token; 4 tokens per 256-thread workgroup.
template <typename TLog>
__global__ __launch_bounds__(256) void route_logits_kernel(
    const TLog* __restrict__ logits, int64_t T, int E, int64_t ld, int top_k, int renorm,
    const int64_t* __restrict__ expert_map, float* __restrict__ topk_w,
    int32_t* __restrict__ topk_ids) {
    __shared__ __attribute__((aligned(16))) uint32_t s_sel[4][kSelectLds];
    const int w = threadIdx.x >> 6;
    const int64_t t = (int64_t)blockIdx.x * 4 + w;
    if (t >= T) return;
    const int lane = threadIdx.x & 63;
    float v[kMaxM];
#pragma unroll
    for (int q = 0; q < kMaxM; ++q) {
        int e = lane + 64 * q;
        v[q] = e < E ? load_logit<TLog>(logits, t * ld + e) : 0.0f;
    }
    wave_select(v, E, top_k, renorm, expert_map, topk_w + t * top_k, topk_ids + t * top_k,
                s_sel[w]);
}

// E <= 128: one token per 256-thread workgroup. The same selection as wave_select's rank
// path with the rank counts split over the four wavefronts (wavefront w compares against keys
// [32w, 32w + 32)); the integer partial ranks are then summed, so the slots are the same.
template <typename TLog>
__global__ __launch_bounds__(256) void route_rank_kernel(
    const TLog* __restrict__ logits, int E, int64_t ld, int top_k, int renorm,
    const int64_t* __restrict__ expert_map, float* __restrict__ topk_w,
    int32_t* __restrict__ topk_ids) {
#pragma clang fp contract(off)
    __shared__ uint64_t s_keys[128];
    __shared__ int s_rank[4][128];
    __shared__ uint32_t s_slots[2 * 64];
    const int w = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t t = blockIdx.x;
    const int nq = (E + 63) >> 6;
    float v[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int e = lane + 64 * q;
        v[q] = e < E ? load_logit<TLog>(logits, t * ld + e) : -__builtin_huge_valf();
    }
    float m = wave_max(fmaxf(v[0], v[1]));
    float part = 0.0f;
    uint64_t mine[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int e = lane + 64 * q;
        const bool in = e < E;
        if (q < nq) {
            const float pe = router_expf(v[q] - m);
            v[q] = in ? pe : -__builtin_huge_valf();
            part = in ? part + pe : part;
        }
        mine[q] = in ? ((uint64_t)(__float_as_uint(v[q]) ^ 0x80000000u) << 32) | (uint32_t)~e : 0;
        if (w == 0 && q < nq) s_keys[e] = mine[q];
    }
    __syncthreads();
    const int n = 64 * nq;
    int r[2][2] = {{0, 0}, {0, 0}};
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
        const int e2 = w * (n / 4) + j;
        if (j < n / 4) {
            const uint64_t k0 = s_keys[e2], k1 = s_keys[e2 + 1];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                r[q][0] += k0 > mine[q] ? 1 : 0;
                r[q][1] += k1 > mine[q] ? 1 : 0;
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) s_rank[w][lane + 64 * q] = r[q][0] + r[q][1];
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int e = lane + 64 * q;
        const int rk = s_rank[0][e] + s_rank[1][e] + s_rank[2][e] + s_rank[3][e];
        if (q < nq && e < E && rk < top_k) {
            s_slots[2 * rk] = __float_as_uint(v[q]);
            s_slots[2 * rk + 1] = (uint32_t)e;
        }
    }
    wave_lds_sync();
    float sel_sum = 0.0f;
    for (int s = 0; s < top_k; ++s) sel_sum = sel_sum + __uint_as_float(s_slots[2 * s]);
    const float denom = renorm ? sel_sum : wave_sum_butterfly(part);
    if (lane < top_k) {
        const int my_i = (int)s_slots[2 * lane + 1];
        topk_w[t * top_k + lane] = __uint_as_float(s_slots[2 * lane]) / denom;
        topk_ids[t * top_k + lane] = expert_map ? (int32_t)expert_map[my_i] : (int32_t)my_i;
    }
}

template <typename TLog>
void launch_route_logits(const TLog* logits, int64_t T, int E, int64_t ld, int top_k, int renorm,
                         const int64_t* expert_map, float* w, int32_t* ids, hipStream_t stream) {
    if (E <= 128)
        hipLaunchKernelGGL(route_rank_kernel<TLog>, dim3((unsigned)T), dim3(256), 0, stream,
                           logits, E, ld, top_k, renorm, expert_map, w, ids);
    else
        hipLaunchKernelGGL(route_logits_kernel<TLog>, dim3((unsigned)((T + 3) / 4)), dim3(256),
                           0, stream, logits, T, E, ld, top_k, renorm, expert_map, w, ids);
}

// Eight consecutive inputs (16 bytes of bf16 or 32 bytes of fp32), kept raw until used.
template <typename TIn>
struct Chunk8;
template <>
struct Chunk8<bf16_t> {
    u32x4 v;
    __device__ __forceinline__ void load(const bf16_t* p) { v = *reinterpret_cast<const u32x4*>(p); }
    __device__ __forceinline__ void zero() { v = u32x4{0u, 0u, 0u, 0u}; }
    __device__ __forceinline__ float get(int i) const {
        return (i & 1) ? hi_bf16(v[i >> 1]) : lo_bf16(v[i >> 1]);
    }
};
template <>
struct Chunk8<float> {
    float4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = reinterpret_cast<const float4*>(p)[0];
        b = reinterpret_cast<const float4*>(p)[1];
    }
    __device__ __forceinline__ void zero() { a = b = make_float4(0.f, 0.f, 0.f, 0.f); }
    __device__ __forceinline__ float get(int i) const {
        const float4& h = i < 4 ? a : b;
        switch (i & 3) {
            case 0: return h.x;
            case 1: return h.y;
            case 2: return h.z;
            default: return h.w;
        }
    }
};

// Combines per-lane partials of N (power of two) different sums in one pass: at distance
// s = 32, 16, ... a lane keeps half of its sums and adds its partner's values for them, until one
// sum is left, then finishes with the plain butterfly. Partners are paired in exactly the order
// of wave_sum_butterfly, so each result is bit-identical to butterflying that sum alone. Lane l
// ends with the full sum number (l >> (6 - log2 N)).
template <int N>
__device__ __forceinline__ float wave_reduce_scatter(float (&acc)[N]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int step = 0; step < 6; ++step) {
        const int s = 32 >> step;
        const int n = (N >> step) > 0 ? (N >> step) : 1;  // sums held before this step
        if (n > 1) {
            // lane-dependent choice made with bit masks on the values (a select between two
            // array elements would become a dynamically indexed array in scratch memory)
            const uint32_t up = (lane & s) ? 0xffffffffu : 0u;
#pragma unroll
            for (int k = 0; k < N / 2; ++k) {
                if (k < n / 2) {
                    const uint32_t lo = __float_as_uint(acc[k]);
                    const uint32_t hi = __float_as_uint(acc[k + n / 2]);
                    const float send = __uint_as_float((lo & up) | (hi & ~up));
                    const float keep = __uint_as_float((hi & up) | (lo & ~up));
                    acc[k] = keep + __shfl_xor(send, s);
                }
            }
        } else {
            acc[0] += __shfl_xor(acc[0], s);
        }
    }
    return acc[0];
}

// Gate GEMM + routing for decode-sized batches: one workgroup of kRouterWaves wavefronts per
// token. Wavefront w computes the per-lane partials of experts e = w + kRouterWaves*j (j < EPW),
// holding x as fp32 in registers and streaming each gate row from L2 (one 16-byte load per lane
// per 512 columns, GE experts in flight), combines its EPW sums with one reduce-scatter, and
// wavefront 0 then selects from the logits in LDS.
template <typename TIn, int NC, int EPW>
__global__ __launch_bounds__(kRouterWaves * 64) void router_kernel(
    const TIn* __restrict__ x, const TIn* __restrict__ gw, int H, int E, int top_k,
    int renorm, const int64_t* __restrict__ expert_map, const float* __restrict__ bias,
    int logits_bf16, float* __restrict__ logits_out, float* __restrict__ topk_w,
    int32_t* __restrict__ topk_ids) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float s_logits[64 * kMaxM];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t t = blockIdx.x;

    float xr[NC * 8];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int h0 = c * 512 + lane * 8;
        Chunk8<TIn> ch;
        ch.zero();
        if (h0 < H) ch.load(x + t * H + h0);
#pragma unroll
        for (int i = 0; i < 8; ++i) xr[c * 8 + i] = ch.get(i);
    }

    constexpr int kWords = sizeof(TIn) * 2;  // VGPRs per raw 8-element chunk
    constexpr int kGe = (96 - NC * 8) / (NC * kWords);
    constexpr int GE0 = kGe < 1 ? 1 : (kGe > 4 ? 4 : kGe);
    constexpr int GE = GE0 > EPW ? EPW : GE0;
    float acc[EPW];
#pragma unroll
    for (int j0 = 0; j0 < EPW; j0 += GE) {
        Chunk8<TIn> gc[GE][NC];
#pragma unroll
        for (int j = 0; j < GE; ++j) {
            const int e = wave + kRouterWaves * (j0 + j);
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int h0 = c * 512 + lane * 8;
                gc[j][c].zero();
                if (e < E && h0 < H) gc[j][c].load(gw + (int64_t)e * H + h0);
            }
        }
#pragma unroll
        for (int j = 0; j < GE; ++j) {
            float a = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                if (c * 512 + lane * 8 < H) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) a = __builtin_fmaf(xr[c * 8 + i], gc[j][c].get(i), a);
                }
            }
            acc[j0 + j] = a;
        }
    }
    float l = wave_reduce_scatter<EPW>(acc);
    constexpr int kShift = (EPW >= 64) ? 0 : (EPW == 32 ? 1 : EPW == 16 ? 2 : EPW == 8 ? 3
                                                          : EPW == 4 ? 4 : EPW == 2 ? 5 : 6);
    const int e = wave + kRouterWaves * (lane >> kShift);
    if ((lane & ((1 << kShift) - 1)) == 0 && e < E) {
        if (bias) l = l + bias[e];
        if (logits_bf16) l = round_bf16(l);
        s_logits[e] = l;
        if (logits_out) logits_out[t * E + e] = l;
    }
    __syncthreads();

    if (wave == 0) {
        float v[kMaxM];
#pragma unroll
        for (int q = 0; q < kMaxM; ++q) {
            int ee = lane + 64 * q;
            v[q] = ee < E ? s_logits[ee] : 0.0f;
        }
        wave_select(v, E, top_k, renorm, expert_map, topk_w + t * top_k, topk_ids + t * top_k,
                    reinterpret_cast<uint32_t*>(s_logits));
    }
}

// Decode-sized batches with a logits buffer: the gate GEMM spread over (token, expert slice)
// workgroups, so the gate matrix is read by many CUs at once instead of by one CU per token.
// Wavefront w of slice s owns experts (s * WAVES + w) * EPW + j, j < EPW; the per-lane fma
// chains and the reduce-scatter are those of router_kernel, so every logit is bit-identical.
// Selection then runs from the buffer.
template <typename TIn, int NC, int EPW, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void router_split_kernel(
    const TIn* __restrict__ x, const TIn* __restrict__ gw, int H, int E,
    const float* __restrict__ bias, int logits_bf16, float* __restrict__ logits) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t t = blockIdx.x;
    const int e0 = (blockIdx.y * WAVES + wave) * EPW;
    if (e0 >= E) return;

    Chunk8<TIn> xc[NC], gc[EPW][NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int h0 = c * 512 + lane * 8;
        xc[c].zero();
        if (h0 < H) xc[c].load(x + t * H + h0);
#pragma unroll
        for (int j = 0; j < EPW; ++j) {
            gc[j][c].zero();
            if (e0 + j < E && h0 < H) gc[j][c].load(gw + (int64_t)(e0 + j) * H + h0);
        }
    }
    float acc[EPW];
#pragma unroll
    for (int j = 0; j < EPW; ++j) {
        float a = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (c * 512 + lane * 8 < H) {
#pragma unroll
                for (int i = 0; i < 8; ++i) a = __builtin_fmaf(xc[c].get(i), gc[j][c].get(i), a);
            }
        }
        acc[j] = a;
    }
    float l = wave_reduce_scatter<EPW>(acc);
    constexpr int kShift = EPW == 1 ? 6 : EPW == 2 ? 5 : EPW == 4 ? 4 : 3;
    const int e = e0 + (lane >> kShift);
    if ((lane & ((1 << kShift) - 1)) == 0 && e < E) {
        if (bias) l = l + bias[e];
        if (logits_bf16) l = round_bf16(l);
        logits[t * E + e] = l;
    }
}

// Large batches: the same logits (identical per-lane fma chains, identical addition tree) computed
// for a tile of 8 tokens x 8 experts per wavefront. Lane j accumulates its 32-element partial for
// all 64 (token, expert) pairs; the 64 x 64 partials are then combined by a transposed
// reduce-scatter (at distance s = 32, 16, ..., 1 each lane keeps half of its pairs and adds the
// partner's values for them), which pairs lanes exactly as wave_sum_butterfly does, so every sum
// is bit-identical to the per-pair butterfly while costing about two shuffles per pair instead of
// six. The 8 tokens' x rows are staged in LDS; each gate row streamed from L2 serves 8 tokens.
constexpr int kTT = 8;   // tokens per workgroup
constexpr int kEG = 8;   // experts per wavefront group
constexpr int kTileWaves = 8;

template <typename TIn, int NC>
__global__ __launch_bounds__(kTileWaves * 64) void router_tile_kernel(
    const TIn* __restrict__ x, const TIn* __restrict__ gw, int64_t T, int H, int E, int top_k,
    int renorm, const int64_t* __restrict__ expert_map, const float* __restrict__ bias,
    int logits_bf16, float* __restrict__ logits_out, float* __restrict__ topk_w,
    int32_t* __restrict__ topk_ids) {
#pragma clang fp contract(off)
    constexpr int W = NC * 512;
    // x rows converted to fp32 once here, so the inner loop does no conversions for them
    __shared__ __attribute__((aligned(16))) float s_x[kTT * W];
    __shared__ __attribute__((aligned(16))) float s_logits[kTT * 512];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t t0 = (int64_t)blockIdx.x * kTT;

    for (int idx = threadIdx.x; idx < kTT * W / 8; idx += kTileWaves * 64) {
        const int tb = idx / (W / 8), h = (idx % (W / 8)) * 8;
        Chunk8<TIn> ch;
        ch.zero();
        if (t0 + tb < T && h < H) ch.load(x + (t0 + tb) * H + h);
        float4 lo, hi;
        lo.x = ch.get(0); lo.y = ch.get(1); lo.z = ch.get(2); lo.w = ch.get(3);
        hi.x = ch.get(4); hi.y = ch.get(5); hi.z = ch.get(6); hi.w = ch.get(7);
        *reinterpret_cast<float4*>(s_x + tb * W + h) = lo;
        *reinterpret_cast<float4*>(s_x + tb * W + h + 4) = hi;
    }
    __syncthreads();

    const int groups = (E + kEG - 1) / kEG;
    for (int grp = wave; grp < groups; grp += kTileWaves) {
        float acc[kTT * kEG];  // pair p = tt * kEG + ee
#pragma unroll
        for (int pi = 0; pi < kTT * kEG; ++pi) acc[pi] = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int h0 = c * 512 + lane * 8;
            if (h0 < H) {
                float g[kEG][8];
#pragma unroll
                for (int ee = 0; ee < kEG; ++ee) {
                    const int e = grp * kEG + ee;
                    Chunk8<TIn> ch;
                    ch.zero();
                    if (e < E) ch.load(gw + (int64_t)e * H + h0);
#pragma unroll
                    for (int i = 0; i < 8; ++i) g[ee][i] = ch.get(i);
                }
#pragma unroll
                for (int tt = 0; tt < kTT; ++tt) {
                    const float4 x0 = *reinterpret_cast<const float4*>(s_x + tt * W + h0);
                    const float4 x1 = *reinterpret_cast<const float4*>(s_x + tt * W + h0 + 4);
                    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int ee = 0; ee < kEG; ++ee)
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            acc[tt * kEG + ee] = __builtin_fmaf(xv[i], g[ee][i], acc[tt * kEG + ee]);
                }
            }
        }
        // transposed reduce-scatter: lane l ends with the sum of pair p == l
        float l = wave_reduce_scatter<kTT * kEG>(acc);
        const int tt = lane / kEG, e = grp * kEG + lane % kEG;
        if (e < E) {
            if (bias) l = l + bias[e];
            if (logits_bf16) l = round_bf16(l);
            s_logits[tt * 512 + e] = l;
            if (logits_out && t0 + tt < T) logits_out[(t0 + tt) * E + e] = l;
        }
    }
    __syncthreads();

    for (int tb = wave; tb < kTT; tb += kTileWaves) {
        const int64_t t = t0 + tb;
        if (t >= T) break;
        float v[kMaxM];
#pragma unroll
        for (int q = 0; q < kMaxM; ++q) {
            int e = lane + 64 * q;
            v[q] = e < E ? s_logits[tb * 512 + e] : 0.0f;
        }
        wave_select(v, E, top_k, renorm, expert_map, topk_w + t * top_k, topk_ids + t * top_k,
                    reinterpret_cast<uint32_t*>(s_logits + tb * 512));
    }
}

// Prefill-sized batches (T > 256, bf16, E <= 128): the gate GEMM on the matrix cores. A
// workgroup of 8 wavefronts owns 64 tokens x all experts; wavefront (wm, wn) computes tokens
// 16 wm .. 16 wm + 15 against experts 64 wn .. 64 wn + 63 with 16x16x32 bf16 MFMAs (fp32
// accumulation), its operands read straight from the row-major x and gate matrices (an MFMA
// operand of a 16-row block is 16 rows x 64 bytes, one 16-byte load per lane), the next k-step's
// operands requested before the current step's MFMAs. The logits go through LDS, are written
// to logits_out (if given) in row order, and each wavefront then routes 8 of the tokens with
// wave_select, the selection every router path uses.
// The MFMA accumulation order is the hardware's, not the fixed order of the other router
// kernels: logits agree with the exact dot products to fp32 accumulation accuracy, and the ids
// and weights are those of the fixed-order selection applied to these logits.
constexpr int kMfmaTokens = 64;
constexpr int kMfmaWaves = 8;
constexpr int kMfmaLd = 128 + 4;  // LDS row stride of the logits tile (floats)
constexpr int kRouterDepth = 4;   // k-steps of operands in flight per wavefront

__global__ __launch_bounds__(kMfmaWaves * 64) void router_mfma_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ gw, int64_t T, int H, int E,
    int top_k, int renorm, const int64_t* __restrict__ expert_map, const float* __restrict__ bias,
    int logits_bf16, float* __restrict__ logits_out, float* __restrict__ topk_w,
    int32_t* __restrict__ topk_ids) {
#pragma clang fp contract(off)
    __shared__ float s_log[kMfmaTokens * kMfmaLd];
    __shared__ __attribute__((aligned(16))) uint32_t s_sel[kMfmaWaves][kSelectLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t t0 = (int64_t)blockIdx.x * kMfmaTokens;

    // operand rows, clamped into range (rows past T or E are computed and never used)
    const int64_t arow = min(t0 + wm * 16 + (lane & 15), T - 1);
    const u32x4* ap = reinterpret_cast<const u32x4*>(x + arow * H + (lane >> 4) * 8);
    const u32x4* bp[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int erow = min(wn * 64 + g * 16 + (lane & 15), E - 1);
        bp[g] = reinterpret_cast<const u32x4*>(gw + (int64_t)erow * H + (lane >> 4) * 8);
    }
    f32x4 acc[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
    // k-steps of 32; one step advances each operand pointer by 32 bf16 (4 x 16 bytes). The
    // operands of kDepth - 1 steps are in flight while a step's MFMAs run (slot s % kDepth);
    // KS is a multiple of kDepth, and the loads past the last step re-read it (unused), so every
    // step issues the same loads and the waits count them exactly.
    const int KS = H / 32;
    u32x4 a[kRouterDepth], b[kRouterDepth][4];
    auto load = [&](int slot_s, int step) {
        step = min(step, KS - 1);
        a[slot_s] = ap[step * 4];
#pragma unroll
        for (int g = 0; g < 4; ++g) b[slot_s][g] = bp[g][step * 4];
    };
#pragma unroll
    for (int d = 0; d + 1 < kRouterDepth; ++d) load(d, d);
    for (int s0 = 0; s0 < KS; s0 += kRouterDepth) {
#pragma unroll
        for (int d = 0; d < kRouterDepth; ++d) {
            load((d + kRouterDepth - 1) % kRouterDepth, s0 + d + kRouterDepth - 1);
            // keep the loads ahead of this step's MFMAs (the scheduler would otherwise sink
            // them next to their uses and shorten the pipeline)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int g = 0; g < 4; ++g)
                acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(a[d]), as_bf16x8(b[d][g]), acc[g], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // element i of block g: token 16 wm + 4 (lane / 16) + i, expert 64 wn + 16 g + lane % 16
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int e = wn * 64 + g * 16 + (lane & 15);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float l = acc[g][i];
            if (bias && e < E) l = l + bias[e];
            if (logits_bf16) l = round_bf16(l);
            s_log[(wm * 16 + (lane >> 4) * 4 + i) * kMfmaLd + e] = l;
        }
    }
    __syncthreads();
    if (logits_out) {
        for (int idx = tid; idx < kMfmaTokens * E; idx += kMfmaWaves * 64) {
            const int tl = idx / E, e = idx - tl * E;
            if (t0 + tl < T) logits_out[(t0 + tl) * E + e] = s_log[tl * kMfmaLd + e];
        }
    }
    constexpr int kPerWave = kMfmaTokens / kMfmaWaves;
    for (int j = 0; j < kPerWave; ++j) {
        const int tl = wave * kPerWave + j;
        const int64_t t = t0 + tl;
        if (t >= T) break;  // uniform across the wavefront
        float v[kMaxM];
#pragma unroll
        for (int q = 0; q < kMaxM; ++q) {
            const int e = lane + 64 * q;
            v[q] = (q < 2 && e < E) ? s_log[tl * kMfmaLd + e] : 0.0f;
        }
        wave_select(v, E, top_k, renorm, expert_map, topk_w + t * top_k, topk_ids + t * top_k,
                    s_sel[wave]);
    }
}

bool router_mfma_supported(int64_t T, int H, int E) {
    return T > 256 && E >= 1 && E <= 128 && H >= 32 * kRouterDepth &&
           H % (32 * kRouterDepth) == 0;
}

hipError_t launch_router_mfma(const void* x, const void* gw, int64_t T, int H, int E, int top_k,
                              int renorm, const int64_t* expert_map, const float* bias,
                              int logits_bf16, float* logits_out, float* w, int32_t* ids,
                              hipStream_t stream) {
    const int64_t blocks = (T + kMfmaTokens - 1) / kMfmaTokens;
    hipLaunchKernelGGL(router_mfma_kernel, dim3((unsigned)blocks), dim3(kMfmaWaves * 64), 0,
                       stream, (const bf16_t*)x, (const bf16_t*)gw, T, H, E, top_k, renorm,
                       expert_map, bias, logits_bf16, logits_out, w, ids);
    return hipGetLastError();
}

template <typename TIn, int NC>
hipError_t launch_router_tile(const void* x, const void* gw, int64_t T, int H, int E, int top_k,
                              int renorm, const int64_t* expert_map, const float* bias,
                              int logits_bf16, float* logits_out, float* w, int32_t* ids,
                              hipStream_t stream) {
    const int64_t blocks = (T + kTT - 1) / kTT;
    hipLaunchKernelGGL((router_tile_kernel<TIn, NC>), dim3((unsigned)blocks),
                       dim3(kTileWaves * 64), 0, stream, (const TIn*)x, (const TIn*)gw, T, H, E,
                       top_k, renorm, expert_map, bias, logits_bf16, logits_out, w, ids);
    return hipGetLastError();
}

template <typename TIn, int NC, int EPW>
hipError_t launch_router_decode(const void* x, const void* gw, int64_t T, int H, int E, int top_k,
                                int renorm, const int64_t* expert_map, const float* bias,
                                int logits_bf16, float* logits_out, float* w, int32_t* ids,
                                hipStream_t stream) {
    hipLaunchKernelGGL((router_kernel<TIn, NC, EPW>), dim3((unsigned)T), dim3(kRouterWaves * 64),
                       0, stream, (const TIn*)x, (const TIn*)gw, H, E, top_k, renorm,
                       expert_map, bias, logits_bf16, logits_out, w, ids);
    return hipGetLastError();
}

template <typename TIn, int NC>
hipError_t launch_router_split(const void* x, const void* gw, int64_t T, int H, int E,
                               int top_k, int renorm, const int64_t* expert_map,
                               const float* bias, int logits_bf16, float* logits, float* w,
                               int32_t* ids, hipStream_t stream) {
    constexpr int kW = 4;
    if (T <= 8) {
        hipLaunchKernelGGL((router_split_kernel<TIn, NC, 1, kW>),
                           dim3((unsigned)T, (unsigned)((E + kW - 1) / kW)), dim3(kW * 64), 0,
                           stream, (const TIn*)x, (const TIn*)gw, H, E, bias, logits_bf16, logits);
    } else {
        // one token per workgroup: tiling tokens (each gate row serving several) measured no
        // faster at decode sizes, where the launch is latency-bound rather than L2-bound
        hipLaunchKernelGGL((router_split_kernel<TIn, NC, 2, kW>),
                           dim3((unsigned)T, (unsigned)((E + 2 * kW - 1) / (2 * kW))),
                           dim3(kW * 64), 0, stream, (const TIn*)x, (const TIn*)gw, H, E, bias,
                           logits_bf16, logits);
    }
    launch_route_logits<float>(logits, T, E, E, top_k, renorm, expert_map, w, ids, stream);
    return hipGetLastError();
}

// Decode-sized batches: one token per workgroup (more workgroups, lower latency), experts per
// wavefront rounded up to a power of two. Larger batches: 8-token tiles.
template <typename TIn, int NC>
hipError_t launch_router_nc(const void* x, const void* gw, int64_t T, int H, int E, int top_k,
                            int renorm, const int64_t* expert_map, const float* bias,
                            int logits_bf16, float* logits_out, float* w, int32_t* ids,
                            hipStream_t stream) {
    if (T > 256)
        return launch_router_tile<TIn, NC>(x, gw, T, H, E, top_k, renorm, expert_map, bias,
                                           logits_bf16, logits_out, w, ids, stream);
    if (logits_out && T <= kSplitMaxT)
        return launch_router_split<TIn, NC>(x, gw, T, H, E, top_k, renorm, expert_map, bias,
                                            logits_bf16, logits_out, w, ids, stream);
    const int epw = (E + kRouterWaves - 1) / kRouterWaves;
#define TSM_DEC(N)                                                                             \
    if (epw <= N)                                                                              \
        return launch_router_decode<TIn, NC, N>(x, gw, T, H, E, top_k, renorm, expert_map,     \
                                                bias, logits_bf16, logits_out, w, ids, stream);
    TSM_DEC(1)
    TSM_DEC(2)
    TSM_DEC(4)
    TSM_DEC(8)
    TSM_DEC(16)
    TSM_DEC(32)
#undef TSM_DEC
    return hipErrorInvalidValue;
}

template <typename TIn>
hipError_t launch_router(const void* x, const void* gw, int64_t T, int H, int E, int top_k,
                         int renorm, const int64_t* expert_map, const float* bias,
                         int logits_bf16, float* logits_out, float* w, int32_t* ids,
                         hipStream_t stream) {
    const int nc = (H + 511) / 512;
#define TSM_ROUTER_NC(N)                                                                         \
    if (nc <= N)                                                                                 \
        return launch_router_nc<TIn, N>(x, gw, T, H, E, top_k, renorm, expert_map, bias,        \
                                        logits_bf16, logits_out, w, ids, stream);
    TSM_ROUTER_NC(1)
    TSM_ROUTER_NC(2)
    TSM_ROUTER_NC(4)
    TSM_ROUTER_NC(8)
#undef TSM_ROUTER_NC
    return hipErrorInvalidValue;
}

int check_route_args(int64_t T, int E, int top_k) {
    TSM_REQUIRE(T >= 0, TSM_E_ARG, "T must be >= 0 (got %lld)", (long long)T);
    TSM_REQUIRE(E >= 1 && E <= 64 * kMaxM, TSM_E_SHAPE, "E must be in [1, %d] (got %d)",
                64 * kMaxM, E);
    TSM_REQUIRE(top_k >= 1 && top_k <= E && top_k <= 64, TSM_E_ARG,
                "top_k must be in [1, min(E, 64)] (got %d, E=%d)", top_k, E);
    return TSM_OK;
}

}  // namespace
}  // namespace tsm

using namespace tsm;

extern "C" int tsm_moe_route(const void* logits, int logits_dtype, int64_t T, int E, int64_t ld,
                             int top_k, int renorm, const int64_t* expert_map, float* topk_w,
                             int32_t* topk_ids, hipStream_t stream) {
    clear_error();
    int rc = check_route_args(T, E, top_k);
    if (rc) return rc;
    TSM_REQUIRE(ld >= E, TSM_E_ARG, "ld (%lld) must be >= E (%d)", (long long)ld, E);
    if (T == 0) return TSM_OK;
    TSM_REQUIRE(logits && topk_w && topk_ids, TSM_E_ARG, "null pointer argument");
    if (logits_dtype == TSM_F32) {
        launch_route_logits<float>((const float*)logits, T, E, ld, top_k, renorm, expert_map,
                                   topk_w, topk_ids, stream);
    } else if (logits_dtype == TSM_BF16) {
        launch_route_logits<bf16_t>((const bf16_t*)logits, T, E, ld, top_k, renorm, expert_map,
                                    topk_w, topk_ids, stream);
    } else {
        set_error("logits dtype code %d not supported", logits_dtype);
        return TSM_E_DTYPE;
    }
    return check_launch("route_logits_kernel");
}

extern "C" int tsm_moe_router(const void* x, const void* gate_w, int dtype, int64_t T, int H,
                              int E, int top_k, int renorm, const int64_t* expert_map,
                              const float* bias, int logits_bf16, float* logits_out,
                              float* topk_w, int32_t* topk_ids, hipStream_t stream) {
    clear_error();
    int rc = check_route_args(T, E, top_k);
    if (rc) return rc;
    TSM_REQUIRE(H >= 8 && H % 8 == 0 && H <= 4096, TSM_E_SHAPE,
                "router needs H %% 8 == 0 and 8 <= H <= 4096 (got %d)", H);
    if (T == 0) return TSM_OK;
    TSM_REQUIRE(x && gate_w && topk_w && topk_ids, TSM_E_ARG, "null pointer argument");
    TSM_REQUIRE(tsm_aligned(16, {x, gate_w}), TSM_E_ARG, "x and gate_w must be 16-byte aligned");
    hipError_t err;
    if (dtype == TSM_BF16 && router_mfma_supported(T, H, E))
        err = launch_router_mfma(x, gate_w, T, H, E, top_k, renorm, expert_map, bias,
                                 logits_bf16, logits_out, topk_w, topk_ids, stream);
    else if (dtype == TSM_BF16)
        err = launch_router<bf16_t>(x, gate_w, T, H, E, top_k, renorm, expert_map, bias,
                                    logits_bf16, logits_out, topk_w, topk_ids, stream);
    else if (dtype == TSM_F32)
        err = launch_router<float>(x, gate_w, T, H, E, top_k, renorm, expert_map, bias,
                                   logits_bf16, logits_out, topk_w, topk_ids, stream);
    else {
        set_error("router dtype code %d not supported", dtype);
        return TSM_E_DTYPE;
    }
    return launch_status(err, "router kernels");
}
