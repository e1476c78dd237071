// MFMA-tiled expert weight layout ("packed"): a one-time reordering of w13 / w2 so that the
// operand of one 16x16x32 MFMA k-step for one 16-row block is 1 KiB of contiguous memory, in the
// order the 64 lanes of a wavefront consume it:
//   packed[e][blk][s][lane][i] = W[e][16*src(blk) + lane%16][32*s + 8*(lane/16) + i]
// (lane < 64, i < 8, s < K/32). For w13 ([E, 2I, H]) the gate and up blocks are interleaved,
// src(2j) = j (gate rows 16j..16j+15) and src(2j+1) = I/16 + j (the matching up rows), so the
// weights one gate_up workgroup streams are contiguous; for w2 ([E, H, I]) src(blk) = blk.
// The packed tensor has the same size as the original.
#include <algorithm>
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

__global__ __launch_bounds__(256) void pack_kernel(const bf16_t* __restrict__ w, int64_t E, int N,
                                                   int K, int interleave,
                                                   bf16_t* __restrict__ out) {
    const int64_t chunks = E * (int64_t)N * K / 8;  // 16-byte chunks
    const int KS = K / 32, NBLK = N / 16;
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < chunks;
         c += (int64_t)gridDim.x * 256) {
        int64_t rest = c;
        const int lane = (int)(rest % 64);
        rest /= 64;
        const int s = (int)(rest % KS);
        rest /= KS;
        const int blk = (int)(rest % NBLK);
        const int64_t e = rest / NBLK;
        const int src = interleave ? ((blk & 1) ? NBLK / 2 + (blk >> 1) : (blk >> 1)) : blk;
        const int row = src * 16 + (lane & 15);
        const int k = s * 32 + (lane >> 4) * 8;
        const u32x4 v = *reinterpret_cast<const u32x4*>(w + (e * N + row) * (int64_t)K + k);
        *reinterpret_cast<u32x4*>(out + c * 8) = v;
    }
}

}  // namespace
}  // namespace tsm

using namespace tsm;

extern "C" int tsm_moe_pack_weights(const void* w, int64_t E, int N, int K, int interleave_halves,
                                    void* out, hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(E >= 1 && N >= 16 && K >= 32 && N % 16 == 0 && K % 32 == 0, TSM_E_SHAPE,
                "pack needs N %% 16 == 0 and K %% 32 == 0 (got E=%lld N=%d K=%d)", (long long)E,
                N, K);
    TSM_REQUIRE(!interleave_halves || N % 32 == 0, TSM_E_SHAPE,
                "interleaved gate/up packing needs N %% 32 == 0");
    TSM_REQUIRE(w && out && w != out, TSM_E_ARG, "pack needs distinct non-null buffers");
    const int64_t chunks = E * (int64_t)N * K / 8;
    const int64_t blocks = std::min<int64_t>((chunks + 255) / 256, 65536);
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       (const bf16_t*)w, E, N, K, interleave_halves, (bf16_t*)out);
    return check_launch("pack_kernel");
}
