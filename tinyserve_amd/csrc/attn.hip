// Attention-side kernels of the qwen3_moe decoder: per-head q/k RMSNorm + rotary embedding with
// the paged KV-cache write, paged causal attention (prefill and decode), and greedy argmax.
//
// Reference: qk_norm_rope / _qk_norm_rope_kernel (tinykernels.py:107-275), paged_attention /
// _paged_attn_kernel / _combine_splits_kernel (tinykernels.py:309-1028), whose results are those
// of serve.py's torch path: RMSNorm (serve.py:799-809), rotary (serve.py:811-814) and
// torch_ref_attention (serve.py:639-688).
//
// KV-cache layout: K pages are [num_pages, page, Hkv, D] as in the reference; V pages are stored
// transposed, [num_pages, Hkv, D, page], so that the P.V product runs on the matrix cores with
// both operands read as they lie (see paged_attn_kernel).
#include <algorithm>
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

// ------------------------------------------------------------------ q/k norm + RoPE + KV write
struct QkArgs {
    bf16_t* q;
    bf16_t* k;
    const bf16_t* v;
    int64_t q_ts, q_hs, k_ts, k_hs, v_ts, v_hs;
    int T, H, Hkv, D;
    const float* cos;  // [T, D/2] rows of stride cs
    const float* sin;
    int64_t cs;
    const bf16_t* qw;  // [D] or null (no per-head norm)
    const bf16_t* kw;
    float eps;
    bf16_t* k_cache;   // [num_pages, page, Hkv, D] or null (no cache write)
    bf16_t* v_cache;   // [num_pages, Hkv, D, page]
    int page;
    int64_t num_slots;     // num_pages * page: slots at or past it are not written
    const int64_t* slots;  // [T] cache slot (page * page_size + offset); < 0: not written
};

// One workgroup per token, one wavefront per head: lane j holds the rotate-half pair (j, j + D/2).
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(QkArgs p) {
#pragma clang fp contract(off)
    const int t = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int half = p.D / 2;
    const bool on = lane < half;
    const float c = on ? p.cos[(int64_t)t * p.cs + lane] : 0.0f;
    const float s = on ? p.sin[(int64_t)t * p.cs + lane] : 0.0f;
    int64_t slot = p.k_cache ? p.slots[t] : -1;
    if (slot >= p.num_slots) slot = -1;
    const int n_rot = p.H + p.Hkv;
    for (int hh = wave; hh < n_rot + (slot >= 0 ? p.Hkv : 0); hh += 4) {
        if (hh >= n_rot) {  // V rows go to the transposed V pages unchanged
            const int kvh = hh - n_rot;
            if (!on) continue;
            const bf16_t* src = p.v + (int64_t)t * p.v_ts + (int64_t)kvh * p.v_hs;
            const int64_t pg = slot / p.page, off = slot % p.page;
            bf16_t* dst = p.v_cache + ((pg * p.Hkv + kvh) * p.D) * p.page + off;
            dst[(int64_t)lane * p.page] = src[lane];
            dst[(int64_t)(lane + half) * p.page] = src[lane + half];
            continue;
        }
        const bool is_q = hh < p.H;
        const int head = is_q ? hh : hh - p.H;
        bf16_t* x = is_q ? p.q + (int64_t)t * p.q_ts + (int64_t)head * p.q_hs
                         : p.k + (int64_t)t * p.k_ts + (int64_t)head * p.k_hs;
        const bf16_t* w = is_q ? p.qw : p.kw;
        float x1 = on ? bf16_to_f32(x[lane]) : 0.0f;
        float x2 = on ? bf16_to_f32(x[lane + half]) : 0.0f;
        if (w) {  // per-head RMSNorm (Qwen3), rounded to bf16 as the reference hands it on
            const float ss = wave_sum_butterfly(x1 * x1 + x2 * x2);
            const float rstd = 1.0f / __builtin_sqrtf(ss / (float)p.D + p.eps);
            if (on) {
                x1 = round_bf16(x1 * rstd * bf16_to_f32(w[lane]));
                x2 = round_bf16(x2 * rstd * bf16_to_f32(w[lane + half]));
            }
        }
        if (!on) continue;
        const bf16_t o1 = f32_to_bf16(x1 * c - x2 * s);
        const bf16_t o2 = f32_to_bf16(x2 * c + x1 * s);
        x[lane] = o1;
        x[lane + half] = o2;
        if (!is_q && slot >= 0) {
            bf16_t* dst = p.k_cache + (slot * p.Hkv + head) * p.D;
            dst[lane] = o1;
            dst[lane + half] = o2;
        }
    }
}

// ------------------------------------------------------------------ paged attention
struct AttnArgs {
    const bf16_t* q;       // [T, H, D] (strided)
    const bf16_t* k_cache; // [num_pages, page, Hkv, D]
    const bf16_t* v_cache; // [num_pages, Hkv, D, page]
    bf16_t* out;           // [T, H, D] (strided)
    int64_t q_ts, q_hs, o_ts, o_hs;
    const int32_t* qsl;    // [B + 1] query_start_loc
    const int32_t* cu_k;   // [B + 1] prefix sums of the context lengths
    const int32_t* bt;     // [B, bt_stride] block table
    int64_t bt_stride;
    int B, Hkv, page;
    int64_t T;             // query rows: requests reaching past them are skipped
    int64_t num_pages;     // page indices are clamped into [0, num_pages)
    float scale_log2;      // softmax scale * log2(e)
    int H;                 // query heads
    // split-KV decode (gridDim.z splits > 1): per (request, head, split) the split's normalised
    // output [B, H, S, D] and its log2-domain log-sum-exp [B, H, S], merged by
    // attn_combine_kernel
    float* part;
    float* lse;
    int splits;            // >= 1: the decode launch's gridDim.z
};

// The decode kernel's and the combine kernel's common test: a request taken by the decode
// launch (one query token, consistent metadata).
__device__ __forceinline__ bool decode_request(const AttnArgs& p, int b, int& q_start,
                                               int& kv_len) {
    q_start = p.qsl[b];
    const int q_len = p.qsl[b + 1] - q_start;
    kv_len = p.cu_k[b + 1] - p.cu_k[b];
    return q_len == 1 && q_start >= 0 && q_start + 1 <= p.T && kv_len >= 1;
}

// Page of context position `pos` (< kv_len): the block-table entry, clamped into the pool, so
// that inconsistent metadata reads a wrong page rather than memory outside the caches.
__device__ __forceinline__ int64_t page_of(const int32_t* bt_row, int pos, const AttnArgs& p) {
    const int64_t col = min((int64_t)(pos / p.page), p.bt_stride - 1);
    const int64_t pg = bt_row[col];
    return pg < 0 ? 0 : (pg >= p.num_pages ? p.num_pages - 1 : pg);
}

constexpr int kAttnWaves = 4;

__device__ __forceinline__ float xor_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    return fmaxf(v, __shfl_xor(v, 32));
}

// Each wavefront owns 16 query rows, a row being one (query token, query head) pair of the KV
// head's group (token-major: row r is token r / GROUP, head GROUP * kvh + r % GROUP), and runs
// the online-softmax recurrence over 32-key blocks of its request's context:
//   S^T = K Q^T: A = 16 keys x 32 d of the K pages (8 consecutive d of one key per lane, as they
//       lie), B = Q^T (8 consecutive d of one row per lane); two 16-key tiles per block. Lane l
//       then holds the scores of row l % 16 for keys 4 (l / 16) + i of each tile.
//   O^T += V^T P^T: the MFMA's reduction index j = 8 (l / 16) + i stands for key
//       4 (l / 16) + i (i < 4) or 16 + 4 (l / 16) + (i - 4) (i >= 4) of the block, which is the
//       order the lane holds its probabilities in, so B = P^T is those 8 values (bf16) as they
//       are, and A = V^T (d x keys) is two 8-byte reads of 4 consecutive keys from the
//       transposed V pages. The result O^T[d][row] leaves lane l with row l % 16 for
//       d = 16 c + 4 (l / 16) + i, the row whose running max and sum it keeps.
// Keys past the context are read from a valid page and masked: scores to -inf, V values to
// zero (unused cache slots may hold anything, and 0 * NaN would be NaN).
// DECODE: one workgroup per (request with one query token, KV head, split of the context); the
// four wavefronts take every fourth key block of the split's range and their partial (max, sum,
// output) are merged through LDS. With one split the merge is the output; with more (split-KV,
// for batches whose B * Hkv workgroups would leave CUs idle) it is the split's partial result,
// merged by attn_combine_kernel.
// Otherwise: workgroups over query tiles of 4 * 16 / GROUP tokens of requests with two or more
// query tokens; each wavefront stops at its last query's causal bound.
template <int D, int GROUP, bool DECODE>
__global__ __launch_bounds__(kAttnWaves * 64) void paged_attn_kernel(AttnArgs p) {
#pragma clang fp contract(off)
    constexpr int NDS = D / 32;   // d steps of the S MFMAs
    constexpr int NDB = D / 16;   // 16-row d blocks of the output
    constexpr int TPW = 16 / GROUP;             // query tokens per wavefront
    constexpr int TQ = kAttnWaves * TPW;        // query tokens per workgroup (prefill)
    static_assert(16 % GROUP == 0 && D % 32 == 0, "shape");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, qd = lane >> 4;
    const int kvh = blockIdx.y;

    int b, tile = 0;
    if (DECODE) {
        b = blockIdx.x;
    } else {
        // the request whose tile list holds this block: start(b) = qsl[b] / TQ + b is
        // non-decreasing, take the last b with start(b) <= blockIdx.x
        int lo = 0, hi = p.B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (p.qsl[mid] / TQ + mid <= (int)blockIdx.x) lo = mid;
            else hi = mid - 1;
        }
        b = lo;
        tile = (int)blockIdx.x - (p.qsl[b] / TQ + b);
    }
    const int q_start = p.qsl[b];
    const int q_len = p.qsl[b + 1] - q_start;
    const int kv_len = p.cu_k[b + 1] - p.cu_k[b];
    if (DECODE ? q_len != 1 : (q_len < 2 || tile * TQ >= q_len)) return;
    // inconsistent metadata (queries outside q, a context shorter than its queries): skipped
    if (q_start < 0 || q_start + q_len > p.T || kv_len < q_len) return;

    const int tok0 = DECODE ? 0 : tile * TQ + wave * TPW;   // this wavefront's first token
    const int tok_r = tok0 + r / GROUP;
    const bool valid_r = tok_r < q_len;
    const int head_r = kvh * GROUP + r % GROUP;
    const int qpos_r = kv_len - q_len + tok_r;
    const int32_t* bt_row = p.bt + (int64_t)b * p.bt_stride;

    // Q^T operand: row r, d = 32 s + 8 qd .. + 7
    u32x4 qop[NDS];
#pragma unroll
    for (int s = 0; s < NDS; ++s) {
        qop[s] = u32x4{0u, 0u, 0u, 0u};
        if (valid_r)
            qop[s] = *reinterpret_cast<const u32x4*>(
                p.q + (int64_t)(q_start + tok_r) * p.q_ts + (int64_t)head_r * p.q_hs + 32 * s +
                8 * qd);
    }

    // key range: prefill wavefronts stop after their last valid query's position
    int kv_end = kv_len;
    if (!DECODE) {
        const int last = min(tok0 + TPW, q_len) - 1;
        kv_end = tok0 < q_len ? kv_len - q_len + last + 1 : 0;
    }
    const int nblk = (kv_end + 31) / 32;
    // split-KV: this workgroup's contiguous range of key blocks (empty ranges report nothing)
    const int nsplit = DECODE ? p.splits : 1, split = DECODE ? (int)blockIdx.z : 0;
    const int chunk = (nblk + nsplit - 1) / nsplit;
    const int blk_lo = split * chunk, blk_hi = min(nblk, blk_lo + chunk);
    const int first = DECODE ? blk_lo + wave : 0, stride = DECODE ? kAttnWaves : 1;

    float m_i = -__builtin_huge_valf(), l_i = 0.0f;
    f32x4 o[NDB];
#pragma unroll
    for (int c = 0; c < NDB; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int64_t kc_tok = (int64_t)p.Hkv * D;

    for (int kb = first; kb < blk_hi; kb += stride) {
        const int key0 = kb * 32;
        // K operand rows (keys key0 + 16 t + r), clamped into the context for the address
        u32x4 kop[2][NDS];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int kc = min(key0 + 16 * t + r, kv_len - 1);
            const int64_t pg = page_of(bt_row, kc, p);
            const bf16_t* src = p.k_cache + (pg * p.page + kc % p.page) * kc_tok + kvh * D + 8 * qd;
#pragma unroll
            for (int s = 0; s < NDS; ++s) kop[t][s] = *reinterpret_cast<const u32x4*>(src + 32 * s);
        }
        // V^T operand: d = 16 c + r, keys key0 + 16 h + 4 qd .. + 3 (one page: page % 4 == 0)
        uint2 vop[2][NDB];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int g = key0 + 16 * h + 4 * qd;
            const int ga = g < kv_len ? g : ((kv_len - 1) & ~3);
            const int64_t pg = page_of(bt_row, ga, p);
            const bf16_t* src =
                p.v_cache + ((pg * p.Hkv + kvh) * D + r) * p.page + ga % p.page;
#pragma unroll
            for (int c = 0; c < NDB; ++c)
                vop[h][c] = *reinterpret_cast<const uint2*>(src + (int64_t)16 * c * p.page);
            // keys past the context: zero
            const int nv = kv_len - g;   // valid keys in this group of 4 (may be <= 0)
            if (nv < 4) {
#pragma unroll
                for (int c = 0; c < NDB; ++c) {
                    uint32_t x0 = vop[h][c].x, x1 = vop[h][c].y;
                    x0 = nv <= 0 ? 0u : nv == 1 ? (x0 & 0xffffu) : x0;
                    x1 = nv <= 2 ? 0u : nv == 3 ? (x1 & 0xffffu) : x1;
                    vop[h][c] = make_uint2(x0, x1);
                }
            }
        }
        // S^T tiles
        f32x4 st[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NDS; ++s)
                st[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kop[t][s]),
                                                                 as_bf16x8(qop[s]), st[t], 0, 0, 0);
        }
        // masked, scaled scores; online softmax for row r
        float sc[2][4];
        float mx = -__builtin_huge_valf();
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = key0 + 16 * t + 4 * qd + i;
                const bool ok = valid_r && key < kv_len && key <= qpos_r;
                sc[t][i] = ok ? st[t][i] * p.scale_log2 : -__builtin_huge_valf();
                mx = fmaxf(mx, sc[t][i]);
            }
        mx = xor_max(mx);
        const float m_new = fmaxf(m_i, mx);
        const float m_use = m_new == -__builtin_huge_valf() ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_i - m_use);
        float pr[2][4];
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pr[t][i] = __builtin_amdgcn_exp2f(sc[t][i] - m_use);
                psum += pr[t][i];
            }
        l_i = l_i * alpha + psum;   // this lane's share of the row sum
        m_i = m_new;
        const u32x4 pop = u32x4{pack_bf16(pr[0][0], pr[0][1]), pack_bf16(pr[0][2], pr[0][3]),
                                pack_bf16(pr[1][0], pr[1][1]), pack_bf16(pr[1][2], pr[1][3])};
#pragma unroll
        for (int c = 0; c < NDB; ++c) {
            o[c] = o[c] * alpha;
            const u32x4 a = u32x4{vop[0][c].x, vop[0][c].y, vop[1][c].x, vop[1][c].y};
            o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(pop), o[c], 0,
                                                            0, 0);
        }
    }
    float l_row = l_i + __shfl_xor(l_i, 16);
    l_row = l_row + __shfl_xor(l_row, 32);

    if (!DECODE) {
        if (!valid_r || tok0 >= q_len) return;
        const float inv = 1.0f / (l_row == 0.0f ? 1.0f : l_row);
        bf16_t* dst = p.out + (int64_t)(q_start + tok_r) * p.o_ts + (int64_t)head_r * p.o_hs;
#pragma unroll
        for (int c = 0; c < NDB; ++c)
            *reinterpret_cast<uint2*>(dst + 16 * c + 4 * qd) =
                make_uint2(pack_bf16(o[c][0] * inv, o[c][1] * inv),
                           pack_bf16(o[c][2] * inv, o[c][3] * inv));
        return;
    }

    // decode: merge the four wavefronts' partial results (fixed order)
    __shared__ float s_m[kAttnWaves][16], s_l[kAttnWaves][16];
    __shared__ float s_o[kAttnWaves][16][D + 4];
    if (qd == 0) {
        s_m[wave][r] = m_i;
        s_l[wave][r] = l_row;
    }
#pragma unroll
    for (int c = 0; c < NDB; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_o[wave][r][16 * c + 4 * qd + i] = o[c][i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < GROUP * D; idx += kAttnWaves * 64) {
        const int row = idx / D, d = idx % D;
        float M = -__builtin_huge_valf();
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, s_m[w][row]);
        const float Mu = M == -__builtin_huge_valf() ? 0.0f : M;
        float L = 0.0f, acc = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float a = __builtin_amdgcn_exp2f(s_m[w][row] - Mu);
            L += a * s_l[w][row];
            acc += a * s_o[w][row][d];
        }
        const int head = kvh * GROUP + row;
        if (nsplit == 1) {
            p.out[(int64_t)q_start * p.o_ts + (int64_t)head * p.o_hs + d] =
                f32_to_bf16(acc / (L == 0.0f ? 1.0f : L));
        } else {
            const int64_t at = ((int64_t)b * p.H + head) * nsplit + split;
            p.part[at * D + d] = L == 0.0f ? 0.0f : acc / L;
            if (d == 0) p.lse[at] = L == 0.0f ? -__builtin_huge_valf() : Mu + log2f(L);
        }
    }
}

// Split-KV merge: one workgroup per (request, query head), a thread per d. The splits' outputs
// are weighted by 2^(lse_s - max lse) in split order (fixed: deterministic), as the reference's
// _combine_splits_kernel (tinykernels.py:801-858) merges them.
template <int D>
__global__ __launch_bounds__(D) void attn_combine_kernel(AttnArgs p) {
    const int b = blockIdx.x, head = blockIdx.y, d = threadIdx.x;
    int q_start, kv_len;
    if (!decode_request(p, b, q_start, kv_len)) return;
    const int S = p.splits;
    const int64_t at0 = ((int64_t)b * p.H + head) * S;
    float M = -__builtin_huge_valf();
    for (int s = 0; s < S; ++s) M = fmaxf(M, p.lse[at0 + s]);
    float W = 0.0f, acc = 0.0f;
    if (M != -__builtin_huge_valf()) {
        for (int s = 0; s < S; ++s) {
            const float w = __builtin_amdgcn_exp2f(p.lse[at0 + s] - M);
            W += w;
            acc += w * p.part[(at0 + s) * D + d];
        }
    }
    p.out[(int64_t)q_start * p.o_ts + (int64_t)head * p.o_hs + d] =
        f32_to_bf16(acc / (W == 0.0f ? 1.0f : W));
}

template <int D, int GROUP>
void launch_attn(const AttnArgs& a, int64_t T, int max_query_len, int splits,
                 hipStream_t stream) {
    hipLaunchKernelGGL((paged_attn_kernel<D, GROUP, true>),
                       dim3((unsigned)a.B, (unsigned)a.Hkv, (unsigned)splits),
                       dim3(kAttnWaves * 64), 0, stream, a);
    if (splits > 1)
        hipLaunchKernelGGL((attn_combine_kernel<D>), dim3((unsigned)a.B, (unsigned)a.H),
                           dim3(D), 0, stream, a);
    if (max_query_len > 1) {
        constexpr int TQ = kAttnWaves * (16 / GROUP);
        const int64_t tiles = T / TQ + a.B;
        hipLaunchKernelGGL((paged_attn_kernel<D, GROUP, false>),
                           dim3((unsigned)tiles, (unsigned)a.Hkv), dim3(kAttnWaves * 64), 0,
                           stream, a);
    }
}

template <int D>
bool launch_attn_d(const AttnArgs& a, int group, int64_t T, int max_query_len, int splits,
                   hipStream_t stream) {
    switch (group) {
        case 1: launch_attn<D, 1>(a, T, max_query_len, splits, stream); return true;
        case 2: launch_attn<D, 2>(a, T, max_query_len, splits, stream); return true;
        case 4: launch_attn<D, 4>(a, T, max_query_len, splits, stream); return true;
        case 8: launch_attn<D, 8>(a, T, max_query_len, splits, stream); return true;
        case 16: launch_attn<D, 16>(a, T, max_query_len, splits, stream); return true;
        default: return false;
    }
}

// ------------------------------------------------------------------ greedy argmax
// One workgroup per row: the largest value, the lowest index among equal values (as
// torch.argmax returns the first maximal index).
template <typename T>
__global__ __launch_bounds__(256) void argmax_kernel(const T* __restrict__ x, int64_t ld, int V,
                                                     int64_t* __restrict__ out) {
    __shared__ float s_v[256];
    __shared__ int s_i[256];
    const int64_t row = blockIdx.x;
    float bv = -__builtin_huge_valf();
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < V; i += 256) {
        float v;
        if constexpr (sizeof(T) == 2) v = bf16_to_f32(x[row * ld + i]);
        else v = x[row * ld + i];
        if (v > bv || bi == 0x7fffffff) {  // ascending i: ties keep the earlier index
            bv = v;
            bi = i;
        }
    }
    s_v[threadIdx.x] = bv;
    s_i[threadIdx.x] = bi;
    __syncthreads();
    for (int w = 128; w >= 1; w >>= 1) {
        if ((int)threadIdx.x < w) {
            const float ov = s_v[threadIdx.x + w];
            const int oi = s_i[threadIdx.x + w];
            if (ov > s_v[threadIdx.x] || (ov == s_v[threadIdx.x] && oi < s_i[threadIdx.x])) {
                s_v[threadIdx.x] = ov;
                s_i[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[row] = s_i[0];
}

}  // namespace
}  // namespace tsm

using namespace tsm;

extern "C" int tsm_qk_norm_rope(void* q, int64_t T, int H, int64_t q_tok_stride,
                                int64_t q_head_stride, void* k, int Hkv, int64_t k_tok_stride,
                                int64_t k_head_stride, const void* v, int64_t v_tok_stride,
                                int64_t v_head_stride, int D, const float* cos, const float* sin,
                                int64_t cs_stride, const void* q_weight, const void* k_weight,
                                float eps, void* k_cache, void* v_cache, int64_t num_pages,
                                int page, const int64_t* slot_mapping, hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(T >= 0 && T <= 0x7fffffffll && H >= 1 && Hkv >= 1 && H % Hkv == 0, TSM_E_ARG,
                "bad sizes (T=%lld H=%d Hkv=%d)", (long long)T, H, Hkv);
    TSM_REQUIRE(D >= 2 && D <= 128 && D % 2 == 0, TSM_E_SHAPE,
                "head_dim must be even and <= 128 (got %d)", D);
    TSM_REQUIRE((q_weight == nullptr) == (k_weight == nullptr), TSM_E_ARG,
                "q and k norm weights come together");
    TSM_REQUIRE(!k_cache || (v_cache && v && slot_mapping && page >= 1 && num_pages >= 1),
                TSM_E_ARG, "a cache write needs v, both caches, slot_mapping, page >= 1 and "
                "num_pages >= 1");
    if (T == 0) return TSM_OK;
    TSM_REQUIRE(q && k && cos && sin, TSM_E_ARG, "null pointer argument");
    QkArgs a{};
    a.q = (bf16_t*)q;
    a.k = (bf16_t*)k;
    a.v = (const bf16_t*)v;
    a.q_ts = q_tok_stride;
    a.q_hs = q_head_stride;
    a.k_ts = k_tok_stride;
    a.k_hs = k_head_stride;
    a.v_ts = v_tok_stride;
    a.v_hs = v_head_stride;
    a.T = (int)T;
    a.H = H;
    a.Hkv = Hkv;
    a.D = D;
    a.cos = cos;
    a.sin = sin;
    a.cs = cs_stride;
    a.qw = (const bf16_t*)q_weight;
    a.kw = (const bf16_t*)k_weight;
    a.eps = eps;
    a.k_cache = (bf16_t*)k_cache;
    a.v_cache = (bf16_t*)v_cache;
    a.page = page;
    a.num_slots = k_cache ? num_pages * page : 0;
    a.slots = slot_mapping;
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)T), dim3(256), 0, stream, a);
    return check_launch("qk_norm_rope_kernel");
}

namespace {
constexpr int kMaxSplits = 64;

// split-KV workspace: partial outputs [B, H, S, D] fp32, then the log-sum-exps [B, H, S] fp32
size_t attn_part_bytes(int64_t B, int H, int D, int S) {
    return ((size_t)B * H * S * D * sizeof(float) + 255) / 256 * 256;
}
}  // namespace

extern "C" size_t tsm_paged_attention_workspace_size(int num_seqs, int H, int D, int num_splits) {
    if (num_seqs < 0 || H < 1 || D < 1 || num_splits < 1 || num_splits > kMaxSplits) return 0;
    if (num_splits == 1) return 0;
    return attn_part_bytes(num_seqs, H, D, num_splits) +
           (size_t)num_seqs * H * num_splits * sizeof(float);
}

extern "C" int tsm_paged_attention(const void* q, int64_t T, int H, int64_t q_tok_stride,
                                   int64_t q_head_stride, const void* k_cache,
                                   const void* v_cache, int64_t num_pages, int page, int Hkv,
                                   int D,
                                   const int32_t* query_start_loc, const int32_t* cu_seqlens_k,
                                   const int32_t* block_table, int64_t bt_stride, int num_seqs,
                                   int max_query_len, float scale, int num_splits, void* ws,
                                   size_t ws_bytes, void* out, int64_t o_tok_stride,
                                   int64_t o_head_stride, hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(num_splits >= 1 && num_splits <= kMaxSplits, TSM_E_ARG,
                "num_splits must be in [1, %d] (got %d)", kMaxSplits, num_splits);
    TSM_REQUIRE(T >= 0 && T <= 0x7fffffffll && num_seqs >= 0 && num_seqs <= 65535, TSM_E_ARG,
                "bad sizes (T=%lld B=%d)", (long long)T, num_seqs);
    TSM_REQUIRE(Hkv >= 1 && H >= Hkv && H % Hkv == 0, TSM_E_ARG,
                "H (%d) must be a positive multiple of Hkv (%d)", H, Hkv);
    const int group = H / Hkv;
    TSM_REQUIRE(group >= 1 && group <= 16 && 16 % group == 0, TSM_E_SHAPE,
                "query heads per KV head must divide 16 (got %d)", group);
    TSM_REQUIRE(D == 64 || D == 128, TSM_E_SHAPE, "head_dim must be 64 or 128 (got %d)", D);
    TSM_REQUIRE(page >= 4 && page % 4 == 0, TSM_E_SHAPE, "page size must be a multiple of 4");
    TSM_REQUIRE(num_pages >= 1 && bt_stride >= 1, TSM_E_ARG,
                "num_pages and the block-table row stride must be >= 1");
    TSM_REQUIRE(q_head_stride % 8 == 0 && q_tok_stride % 8 == 0 && o_head_stride % 4 == 0 &&
                    o_tok_stride % 4 == 0,
                TSM_E_ARG, "q rows must be 16-byte and out rows 8-byte aligned");
    if (T == 0 || num_seqs == 0) return TSM_OK;
    TSM_REQUIRE(q && k_cache && v_cache && query_start_loc && cu_seqlens_k && block_table && out,
                TSM_E_ARG, "null pointer argument");
    TSM_REQUIRE(tsm_aligned(16, {q, k_cache}) && tsm_aligned(8, {v_cache, out}), TSM_E_ARG,
                "attention needs 16-byte aligned q and K pages, 8-byte aligned V pages and out");
    const size_t need = tsm_paged_attention_workspace_size(num_seqs, H, D, num_splits);
    TSM_REQUIRE(num_splits == 1 || (ws && ws_bytes >= need && tsm_aligned(256, {ws})),
                TSM_E_WORKSPACE,
                "split-KV needs a 256-byte aligned workspace of >= %zu bytes (got %zu)", need,
                ws_bytes);
    AttnArgs a{};
    a.q = (const bf16_t*)q;
    a.k_cache = (const bf16_t*)k_cache;
    a.v_cache = (const bf16_t*)v_cache;
    a.out = (bf16_t*)out;
    a.q_ts = q_tok_stride;
    a.q_hs = q_head_stride;
    a.o_ts = o_tok_stride;
    a.o_hs = o_head_stride;
    a.qsl = query_start_loc;
    a.cu_k = cu_seqlens_k;
    a.bt = block_table;
    a.bt_stride = bt_stride;
    a.B = num_seqs;
    a.Hkv = Hkv;
    a.page = page;
    a.num_pages = num_pages;
    a.T = T;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.H = H;
    a.splits = num_splits;
    if (num_splits > 1) {
        a.part = reinterpret_cast<float*>(ws);
        a.lse = reinterpret_cast<float*>((char*)ws + attn_part_bytes(num_seqs, H, D, num_splits));
    }
    const bool ok =
        D == 128 ? launch_attn_d<128>(a, group, T, max_query_len, num_splits, stream)
                 : launch_attn_d<64>(a, group, T, max_query_len, num_splits, stream);
    TSM_REQUIRE(ok, TSM_E_SHAPE, "no attention kernel for group %d", group);
    return check_launch("paged_attn_kernel");
}

extern "C" int tsm_greedy_argmax(const void* logits, int dtype, int64_t rows, int64_t ld, int V,
                                 int64_t* out, hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(rows >= 0 && rows <= 0x7fffffffll && V >= 1 && ld >= V, TSM_E_ARG,
                "bad sizes (rows=%lld V=%d ld=%lld)", (long long)rows, V, (long long)ld);
    if (rows == 0) return TSM_OK;
    TSM_REQUIRE(logits && out, TSM_E_ARG, "null pointer argument");
    if (dtype == TSM_F32)
        hipLaunchKernelGGL(argmax_kernel<float>, dim3((unsigned)rows), dim3(256), 0, stream,
                           (const float*)logits, ld, V, out);
    else if (dtype == TSM_BF16)
        hipLaunchKernelGGL(argmax_kernel<bf16_t>, dim3((unsigned)rows), dim3(256), 0, stream,
                           (const bf16_t*)logits, ld, V, out);
    else {
        set_error("argmax dtype code %d not supported", dtype);
        return TSM_E_DTYPE;
    }
    return check_launch("argmax_kernel");
}
