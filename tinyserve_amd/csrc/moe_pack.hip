// MFMA-tiled expert weight layout ("packed"): a one-time reordering of w13 / w2 so that the
// operand of one 16x16x32 MFMA k-step for one 16-row block is 1 KiB of contiguous memory, in the
// order the 64 lanes of a wavefront consume it:
//   packed[e][blk][s][lane][i] = W[e][16*src(blk) + lane%16][32*s + 8*(lane/16) + i]
// (lane < 64, i < 8, s < K/32). For w13 ([E, 2I, H]) the gate and up blocks are interleaved,
// src(2j) = j (gate rows 16j..16j+15) and src(2j+1) = I/16 + j (the matching up rows), so the
// weights one gate_up workgroup streams are contiguous; for w2 ([E, H, I]) src(blk) = blk.
// Without padding the packed tensor has the same size as the original; the padded variant
// rounds N and K up to the sizes the tile kernels support and fills the margin with zeros.
#include <algorithm>
#include "common.h"
#include "internal.h"
#include "tinyserve_moe.h"

namespace tsm {
namespace {

// Destination geometry N x K (the padded shape the kernels run at); the source holds
// n_src x k_src of it (w13: n_src = I rows of each half; w2: n_src = H rows), with row pitch
// k_src. Destination elements outside the source are zero, so padded rows and columns contribute
// exact zeros to every product and sum they enter.
__global__ __launch_bounds__(256) void pack_kernel(const bf16_t* __restrict__ w, int64_t E, int N,
                                                   int K, int n_src, int k_src, int interleave,
                                                   bf16_t* __restrict__ out) {
    const int64_t chunks = E * (int64_t)N * K / 8;  // 16-byte chunks
    const int KS = K / 32, NBLK = N / 16;
    const int64_t src_rows = interleave ? 2 * (int64_t)n_src : n_src;  // rows per source expert
    const bool vec = (k_src % 8) == 0;  // source rows are 16-byte aligned
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < chunks;
         c += (int64_t)gridDim.x * 256) {
        int64_t rest = c;
        const int lane = (int)(rest % 64);
        rest /= 64;
        const int s = (int)(rest % KS);
        rest /= KS;
        const int blk = (int)(rest % NBLK);
        const int64_t e = rest / NBLK;
        // row within the destination half (interleaved) or the whole matrix, and the source row
        int row, half = 0;
        if (interleave) {
            half = blk & 1;
            row = (blk >> 1) * 16 + (lane & 15);
        } else {
            row = blk * 16 + (lane & 15);
        }
        const int k = s * 32 + (lane >> 4) * 8;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (row < n_src && k < k_src) {
            const bf16_t* src = w + (e * src_rows + (int64_t)half * n_src + row) * (int64_t)k_src + k;
            if (vec) {
                v = *reinterpret_cast<const u32x4*>(src);
            } else {
                uint16_t h[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) h[i] = k + i < k_src ? src[i] : (uint16_t)0;
                v = u32x4{h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16),
                          h[4] | ((uint32_t)h[5] << 16), h[6] | ((uint32_t)h[7] << 16)};
            }
        }
        *reinterpret_cast<u32x4*>(out + c * 8) = v;
    }
}

}  // namespace
}  // namespace tsm

using namespace tsm;

extern "C" int tsm_moe_padded_shape(int H, int I, int* H_pad, int* I_pad) {
    clear_error();
    TSM_REQUIRE(H >= 1 && I >= 1 && H <= (1 << 20) && I <= (1 << 20), TSM_E_ARG,
                "sizes out of range (H=%d I=%d)", H, I);
    TSM_REQUIRE(H_pad && I_pad, TSM_E_ARG, "null pointer argument");
    // the expert kernels take H % 128 == 0 and I % 64 == 0 (check_moe_shapes)
    *H_pad = H % 128 == 0 ? H : (H + 127) / 128 * 128;
    *I_pad = I % 64 == 0 ? I : (I + 127) / 128 * 128;
    return TSM_OK;
}

extern "C" int tsm_moe_pack_weights_padded(const void* w, int64_t E, int N, int K, int N_pad,
                                           int K_pad, int interleave_halves, void* out,
                                           hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(E >= 1 && N >= 1 && K >= 1 && N_pad >= N && K_pad >= K, TSM_E_SHAPE,
                "pack needs 1 <= N <= N_pad and 1 <= K <= K_pad (got E=%lld N=%d/%d K=%d/%d)",
                (long long)E, N, N_pad, K, K_pad);
    TSM_REQUIRE(N_pad % 16 == 0 && K_pad % 32 == 0, TSM_E_SHAPE,
                "packed shape needs N_pad %% 16 == 0 and K_pad %% 32 == 0 (got %d, %d)", N_pad,
                K_pad);
    TSM_REQUIRE(!interleave_halves || (N % 2 == 0 && N_pad % 32 == 0), TSM_E_SHAPE,
                "interleaved gate/up packing needs an even N and N_pad %% 32 == 0");
    TSM_REQUIRE(w && out && w != out, TSM_E_ARG, "pack needs distinct non-null buffers");
    const int64_t chunks = E * (int64_t)N_pad * K_pad / 8;
    const int64_t blocks = std::min<int64_t>((chunks + 255) / 256, 65536);
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       (const bf16_t*)w, E, N_pad, K_pad, interleave_halves ? N / 2 : N, K,
                       interleave_halves, (bf16_t*)out);
    return check_launch("pack_kernel");
}

extern "C" int tsm_moe_pack_weights(const void* w, int64_t E, int N, int K, int interleave_halves,
                                    void* out, hipStream_t stream) {
    clear_error();
    TSM_REQUIRE(E >= 1 && N >= 16 && K >= 32 && N % 16 == 0 && K % 32 == 0, TSM_E_SHAPE,
                "pack needs N %% 16 == 0 and K %% 32 == 0 (got E=%lld N=%d K=%d)", (long long)E,
                N, K);
    TSM_REQUIRE(!interleave_halves || N % 32 == 0, TSM_E_SHAPE,
                "interleaved gate/up packing needs N %% 32 == 0");
    return tsm_moe_pack_weights_padded(w, E, N, K, N, K, interleave_halves, out, stream);
}
