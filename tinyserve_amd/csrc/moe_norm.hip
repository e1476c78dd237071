// Residual-add RMSNorm, optionally fused with the MoE block's top-k combine.
//
// Reference: the decoder's add_rmsnorm (serve.py:1177-1193) over tinykernels.rmsnorm /
// _rmsnorm_kernel (tinykernels.py:26-105): residual = bf16(float(x) + float(residual)), then
// out = bf16(float(residual) * rsqrt(mean(residual^2) + eps) * float(w)). With the MoE block's
// per-slot rows as x (fused_moe with sum_topk=False, tinykernels.py:1796), x itself is first the
// fixed-order k-sum bf16(sum_s rows[t*k+s]) that tsm_moe_combine computes, so the [T, H] MoE
// output is never written to memory and read back, and one launch replaces two.
//
// One workgroup per token row, 256 threads; each thread owns CH 16-byte chunks of the row. The
// sum of squares is taken in a fixed order (per thread: chunk, then element; then the XOR
// butterfly within each wavefront; then the four wavefront partials in order), so the result is
// deterministic and independent of the batch.
#include <algorithm>
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

constexpr int kThreads = 256;

template <int CH, bool STREAM>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(
    const bf16_t* __restrict__ x, int k, bf16_t* __restrict__ residual, int residual_in,
    const bf16_t* __restrict__ weight, float eps, bf16_t* __restrict__ out, int H) {
    __shared__ float s_part[kThreads / 64];
    const int64_t t = blockIdx.x;
    const int tid = threadIdx.x, cpr = H / 8;
    float v[CH][8];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const int c = tid + j * kThreads;
        if (c >= cpr) {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[j][i] = 0.0f;
            continue;
        }
        // k-sum in fp32 in slot order, rounded once (k = 1: x itself)
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < k; ++s) {
            const u32x4* src = reinterpret_cast<const u32x4*>(x + ((t * k + s) * H + c * 8));
            const u32x4 w = STREAM ? __builtin_nontemporal_load(src) : *src;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] += lo_bf16(w[q]);
                acc[2 * q + 1] += hi_bf16(w[q]);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = round_bf16(acc[i]);
        if (residual) {
            u32x4* rp = reinterpret_cast<u32x4*>(residual + (t * H + c * 8));
            if (residual_in) {
                const u32x4 r = *rp;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[j][2 * q] = round_bf16(v[j][2 * q] + lo_bf16(r[q]));
                    v[j][2 * q + 1] = round_bf16(v[j][2 * q + 1] + hi_bf16(r[q]));
                }
            }
            u32x4 o;
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = pack_bf16(v[j][2 * q], v[j][2 * q + 1]);
            *rp = o;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(v[j][i], v[j][i], ss);
    }
    ss = wave_sum_butterfly(ss);
    if ((tid & 63) == 0) s_part[tid >> 6] = ss;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) total += s_part[w];
    const float rstd = 1.0f / __builtin_sqrtf(total / (float)H + eps);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const int c = tid + j * kThreads;
        if (c >= cpr) continue;
        const u32x4 wv = *reinterpret_cast<const u32x4*>(weight + c * 8);
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o[q] = pack_bf16(v[j][2 * q] * rstd * lo_bf16(wv[q]),
                             v[j][2 * q + 1] * rstd * hi_bf16(wv[q]));
        u32x4* dst = reinterpret_cast<u32x4*>(out + (t * H + c * 8));
        if (STREAM) __builtin_nontemporal_store(o, dst);
        else *dst = o;
    }
}

template <int CH>
void launch_norm(const bf16_t* x, int64_t T, int H, int k, bf16_t* residual, int residual_in,
                 const bf16_t* weight, float eps, bf16_t* out, hipStream_t stream) {
    // rows larger than the L2s of the 8 XCDs stream through with non-temporal accesses
    if ((int64_t)T * k * H * 2 > (32ll << 20))
        hipLaunchKernelGGL((add_rmsnorm_kernel<CH, true>), dim3((unsigned)T), dim3(kThreads), 0,
                           stream, x, k, residual, residual_in, weight, eps, out, H);
    else
        hipLaunchKernelGGL((add_rmsnorm_kernel<CH, false>), dim3((unsigned)T), dim3(kThreads), 0,
                           stream, x, k, residual, residual_in, weight, eps, out, H);
}

}  // namespace
}  // namespace tsm

using namespace tsm;

extern "C" int tsm_add_rmsnorm(const void* x, int64_t T, int H, int top_k, void* residual,
                               int residual_in, const void* weight, float eps, void* out,
                               hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(T >= 0 && T <= 0x7fffffffll, TSM_E_ARG, "T out of range (%lld)", (long long)T);
    TSM_REQUIRE(H >= 8 && H % 8 == 0 && H <= 8 * kThreads * 8, TSM_E_SHAPE,
                "add_rmsnorm needs H %% 8 == 0 and 8 <= H <= %d (got %d)", 8 * kThreads * 8, H);
    TSM_REQUIRE(top_k >= 1 && top_k <= 64, TSM_E_ARG, "top_k must be in [1, 64] (got %d)",
                top_k);
    TSM_REQUIRE(eps >= 0.0f, TSM_E_ARG, "eps must be >= 0");
    TSM_REQUIRE(!residual_in || residual, TSM_E_ARG, "residual_in needs a residual buffer");
    if (T == 0) return TSM_OK;
    TSM_REQUIRE(x && weight && out, TSM_E_ARG, "null pointer argument");
    TSM_REQUIRE(tsm_aligned(16, {x, residual, weight, out}), TSM_E_ARG,
                "add_rmsnorm needs 16-byte aligned tensors");
    const int cpr = H / 8;
    const bf16_t* xb = (const bf16_t*)x;
    bf16_t* rb = (bf16_t*)residual;
    if (cpr <= kThreads)
        launch_norm<1>(xb, T, H, top_k, rb, residual_in, (const bf16_t*)weight, eps,
                       (bf16_t*)out, stream);
    else if (cpr <= 2 * kThreads)
        launch_norm<2>(xb, T, H, top_k, rb, residual_in, (const bf16_t*)weight, eps,
                       (bf16_t*)out, stream);
    else if (cpr <= 4 * kThreads)
        launch_norm<4>(xb, T, H, top_k, rb, residual_in, (const bf16_t*)weight, eps,
                       (bf16_t*)out, stream);
    else
        launch_norm<8>(xb, T, H, top_k, rb, residual_in, (const bf16_t*)weight, eps,
                       (bf16_t*)out, stream);
    return check_launch("add_rmsnorm_kernel");
}
