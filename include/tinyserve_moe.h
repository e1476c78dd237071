/*
 * tinyserve_moe.h - C ABI of the MI355X (gfx950) fused mixture-of-experts operator.
 *
 * Drop-in boundary for tinyserve's qwen3_moe feed-forward block: every entry point here replaces
 * one function of the reference's Python/Triton MoE path (cited per function, file:line into the
 * reference tree). Arguments are plain device pointers, sizes and a hipStream_t; there are no torch
 * types in the signatures. All entry points:
 *   - are asynchronous on `stream` (no host synchronisation, no device allocation, no memset), so
 *     they can be captured into a HIP graph;
 *   - launch a grid whose shape depends only on the sizes, never on the routing;
 *   - return TSM_OK (0) on success, a negative TSM_E* code on invalid arguments (nothing is launched
 *     then), or TSM_E_HIP when a launch fails; tsm_last_error() describes the last failure.
 *
 * Layouts (row-major, contiguous):
 *   x       [T, H]       bf16     activations
 *   gate_w  [E, H]       bf16     router weight (nn.Linear(H, E, bias=False).weight)
 *   w13     [E, 2I, H]   bf16     rows [0, I) = gate_proj, rows [I, 2I) = up_proj
 *   w2      [E, H, I]    bf16     down_proj
 *   topk_w  [T, k]       fp32     routing weights, slot 0 = largest
 *   topk_ids[T, k]       int32    local expert ids, -1 = expert owned by another GPU
 */
#ifndef TINYSERVE_MOE_H
#define TINYSERVE_MOE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TSM_OK = 0,
    TSM_E_ARG = -1,        /* null pointer, negative size, top_k out of range */
    TSM_E_SHAPE = -2,      /* shape the kernels do not support (e.g. H % 64 != 0) */
    TSM_E_DTYPE = -3,      /* dtype code not supported by this entry point */
    TSM_E_WORKSPACE = -4,  /* workspace pointer null/misaligned or smaller than required */
    TSM_E_HIP = -5         /* a HIP launch failed */
};

/* dtype codes */
enum { TSM_F32 = 0, TSM_BF16 = 1 };

/* expert weight layouts */
enum { TSM_LAYOUT_REFERENCE = 0, TSM_LAYOUT_PACKED = 1 };

/* Description of the last error on the calling thread ("" if none). */
const char* tsm_last_error(void);

/* ABI version, bumped on any signature change. */
int tsm_abi_version(void);

/*
 * Routing from precomputed logits.
 * Replaces tinykernels.moe_route / _moe_route_kernel (tinykernels.py:1535-1583), and the torch
 * router branch of SparseMoE.forward (serve.py:1089-1096).
 * logits: [T, E] with row stride `ld` elements, dtype TSM_F32 or TSM_BF16 (converted exactly to
 * fp32). Per token: p_e = exp(l_e - max l) in fp32; the top_k largest p are taken largest first,
 * lowest expert index first among equal p; weights = p / sum(selected p) when renorm != 0, else
 * p / sum(all p). ids are mapped through expert_map (int64 [E], global -> local id or -1) when it
 * is non-null. Requires 1 <= top_k <= min(E, 64), E <= 512.
 */
int tsm_moe_route(const void* logits, int logits_dtype, int64_t T, int E, int64_t ld, int top_k,
                  int renorm, const int64_t* expert_map, float* topk_w, int32_t* topk_ids,
                  hipStream_t stream);

/*
 * Fused router: gate GEMM (fp32 accumulation with a fixed summation order) + optional per-expert
 * fp32 bias + optional rounding of the logits to bf16 + the routing of tsm_moe_route. One launch;
 * with logits_out given and T <= 256, two (the gate GEMM spread over expert slices into
 * logits_out, then the selection from it), which is lower latency at decode sizes.
 * Replaces `self.gate(x)` followed by tk.moe_route in SparseMoE.forward (serve.py:1079-1080).
 * x: [T, H], gate_w: [E, H], both of dtype `dtype` (TSM_BF16 or TSM_F32). bias: [E] fp32 or null.
 * logits_bf16 != 0 rounds each logit to bf16 (round-to-nearest-even) before the softmax, as the
 * reference's bf16 nn.Linear output is. logits_out: [T, E] fp32 or null (the logits the softmax
 * saw). Requires H % 8 == 0, 8 <= H <= 4096, and the tsm_moe_route limits.
 */
int tsm_moe_router(const void* x, const void* gate_w, int dtype, int64_t T, int H, int E,
                   int top_k, int renorm, const int64_t* expert_map, const float* bias,
                   int logits_bf16, float* logits_out, float* topk_w, int32_t* topk_ids,
                   hipStream_t stream);

/*
 * Block-aligned expert permutation.
 * Replaces moe_align_block_size (tinykernels.py:1070-1190) and moe_align_block_size_triton
 * (tinykernels.py:1462-1532); same outputs bit for bit.
 * ids: [numel] int32 (flattened topk_ids); negative ids go to the remote bucket E.
 * Outputs: sorted_ids [tsm_moe_max_padded(numel,E,block_m)] int32, expert_ids
 * [max_padded / block_m] int32, total [1] int32. `ws` is scratch of tsm_moe_align_workspace_size()
 * bytes (may be null when that size is 0).
 */
int64_t tsm_moe_max_padded(int64_t numel, int E, int block_m);
size_t tsm_moe_align_workspace_size(int64_t numel, int E, int block_m);
int tsm_moe_align(const int32_t* ids, int64_t numel, int E, int block_m, int32_t* sorted_ids,
                  int32_t* expert_ids, int32_t* total, void* ws, size_t ws_bytes,
                  hipStream_t stream);

/*
 * out[r, :] = bf16( bf16(silu(gate[r, :])) * up[r, :] ), bf16 tensors, strides in elements.
 * Replaces silu_and_mul / _silu_mul_kernel (tinykernels.py:280-307).
 */
int tsm_silu_and_mul(const void* gate, int64_t gate_stride, const void* up, int64_t up_stride,
                     void* out, int64_t out_stride, int64_t rows, int64_t N, hipStream_t stream);

/*
 * Tile height (rows per expert tile) fused_moe uses for a batch of T tokens with the given weight
 * layout (TSM_LAYOUT_*). The reference picks 16 when T*k <= 4E, else 64 (tinykernels.py:1779);
 * this build picks from its own kernel table: 0 = the expert-major stages below (no tiles, no
 * permutation; T*k <= 12E within their size limits), else 16 (T*k <= 4E) / 64, and 128 for
 * packed weights above 32E. 256 (packed weights) is returned only where tsm_moe_set_block_m
 * installed it.
 */
int tsm_moe_block_m(int64_t T, int H, int I, int E, int top_k, int weight_layout);

/*
 * Install a tile height for the plans of fused_moe / moe_forward with the given weight layout,
 * for assignment counts numel = T * top_k in the power-of-two buckets that [numel_lo, numel_hi]
 * touches (bucket b: 2^b <= numel < 2^(b+1)); block_m = -1 restores the static table there.
 * 0 selects the expert-major stages (used only where their size limits allow), 16 / 64 (and 128
 * or 256 with packed weights, where 2I and H are multiples of 256) the tiled stages. Process-wide; plans already captured in a HIP graph keep
 * their kernels. Workspace sizes follow the installed heights, so query them after installing.
 * The build's counterpart of the autotuning of autotune_fused_moe (tinykernels.py:1798-1811):
 * kernels.autotune_fused_moe times the candidates and installs the fastest.
 */
int tsm_moe_set_block_m(int64_t numel_lo, int64_t numel_hi, int weight_layout, int block_m);

/*
 * Experts on sorted rows: align + grouped gate_up GEMM with the SwiGLU epilogue + grouped down GEMM
 * scaled by the routing weight + (sum_topk) the deterministic fixed-order k-sum.
 * Replaces fused_moe (tinykernels.py:1767-1796) with _moe_gemm/_fused_moe_kernel
 * (tinykernels.py:1589-1765) and silu_and_mul.
 * out: [T, H] bf16 when sum_topk != 0, else [T*k, H] bf16 (row t*k+s = weighted expert output of
 * slot s, zeros for remote slots). Requires H % 128 == 0, I % 64 == 0 (both >= 64).
 */
size_t tsm_fused_moe_workspace_size(int64_t T, int H, int I, int E, int top_k);
int tsm_fused_moe(const void* x, const void* w13, const void* w2, const float* topk_w,
                  const int32_t* topk_ids, int64_t T, int H, int I, int E, int top_k,
                  int sum_topk, void* out, void* ws, size_t ws_bytes, hipStream_t stream);

/*
 * The stages of tsm_fused_moe, for callers that schedule them separately (and for per-kernel
 * timing). Each is one launch of the corresponding stage of _moe_gemm / _fused_moe_kernel
 * (tinykernels.py:1746-1765, 1589-1744) on the outputs of tsm_moe_align for the same block_m
 * (supported: 16, 64; 128 and 256 with packed weights; gate_up at 256 needs x below 4 GiB):
 *   gate_up: act[max_padded, I] (expert-sorted rows) = bf16(bf16(silu(bf16(x W1^T))) *
 *            bf16(x W3^T)) with x gathered as x[sorted_ids[r] / top_k]; rows of remote tiles
 *            are not written.
 *   down:    rows[a, :] = bf16((act[r] W2^T) * topk_w[a]) for a = sorted_ids[r] < numel; zeros
 *            for remote assignments. top_k is 1 for this GEMM (act rows are assignments).
 *   combine: out[t, :] = bf16(sum_{s<k} rows[t*k + s, :]), fp32 accumulation in slot order
 *            (tinykernels.py:1796).
 * weight_layout: TSM_LAYOUT_REFERENCE (w13/w2 as above) or TSM_LAYOUT_PACKED
 * (tsm_moe_pack_weights output).
 */
int tsm_moe_gemm_gate_up(const void* x, const void* w13, const int32_t* sorted_ids,
                         const int32_t* expert_ids, const int32_t* total, int64_t numel,
                         int top_k, int H, int I, int E, int block_m, int weight_layout,
                         void* act, hipStream_t stream);
int tsm_moe_gemm_down(const void* act, const void* w2, const float* topk_w,
                      const int32_t* sorted_ids, const int32_t* expert_ids, const int32_t* total,
                      int64_t numel, int H, int I, int E, int block_m, int weight_layout,
                      void* rows, hipStream_t stream);
int tsm_moe_combine(const void* rows, int64_t T, int H, int top_k, void* out, hipStream_t stream);

/*
 * tsm_fused_moe for fp32 activations and weights (same layouts, fp32 elements): every
 * intermediate in fp32, as the reference's fused_moe keeps them in x.dtype (tinykernels.py:1784-
 * 1791) and moe_reference computes an fp32 layer (serve.py:933-996): act = silu(x W1^T) * (x W3^T),
 * rows = (act W2^T) * topk_w, out = fixed-order fp32 k-sum. Runs on the vector ALUs (16-row
 * expert tiles of the align step); for the tiny fp32 configuration, not for throughput. Any H, I.
 */
size_t tsm_fused_moe_f32_workspace_size(int64_t T, int H, int I, int E, int top_k);
int tsm_fused_moe_f32(const float* x, const float* w13, const float* w2, const float* topk_w,
                      const int32_t* topk_ids, int64_t T, int H, int I, int E, int top_k,
                      int sum_topk, float* out, void* ws, size_t ws_bytes, hipStream_t stream);

/*
 * Expert-major stages used by fused_moe for decode-sized batches (tsm_moe_block_m() == 0): no
 * permutation step; each workgroup finds its expert's assignments by scanning topk_ids [numel]
 * (stable flat order, as moe_align_block_size orders them), and act [numel, I] holds the
 * activations in expert-sorted order (expert e's rows start at the number of assignments to
 * experts < e). gate_up writes act; down writes rows [numel, H] (zeros for ids outside [0, E)).
 * Requires numel <= 4096, H and I multiples of 128 with H/128, I/128 <= 16.
 */
int tsm_moe_expert_gate_up(const void* x, const void* w13, const int32_t* topk_ids,
                           int64_t numel, int top_k, int H, int I, int E, int weight_layout,
                           void* act, hipStream_t stream);
int tsm_moe_expert_down(const void* act, const void* w2, const float* topk_w,
                        const int32_t* topk_ids, int64_t numel, int H, int I, int E,
                        int weight_layout, void* rows, hipStream_t stream);

/*
 * Whole SparseMoE.forward on one GPU (serve.py:1076-1087 at TP=1): fused router then fused_moe.
 * Router options as in tsm_moe_router; topk_w/topk_ids ([T, k]) may be null when the caller does
 * not need them (they then live in the workspace).
 */
size_t tsm_moe_forward_workspace_size(int64_t T, int H, int I, int E, int top_k);
int tsm_moe_forward(const void* x, const void* gate_w, const void* w13, const void* w2,
                    const int64_t* expert_map, const float* bias, int64_t T, int H, int I, int E,
                    int top_k, int renorm, int logits_bf16, int sum_topk, void* out,
                    float* topk_w, int32_t* topk_ids, void* ws, size_t ws_bytes,
                    hipStream_t stream);

/*
 * Residual-add RMSNorm, optionally fused with the MoE block's top-k combine.
 * Replaces the decoder's add_rmsnorm (serve.py:1177-1193) over tinykernels.rmsnorm /
 * _rmsnorm_kernel (tinykernels.py:26-105) and, with top_k > 1, also the k-sum of fused_moe
 * (tinykernels.py:1796) that produced its input.
 * x: [T*top_k, H] bf16 (top_k = 1: the [T, H] input itself; top_k > 1: the per-slot rows of
 * tsm_fused_moe with sum_topk = 0). Per token t:
 *   s = bf16(sum_{j<top_k} x[t*top_k + j])            (fp32, slot order; top_k = 1: x[t])
 *   if residual_in: s = bf16(float(s) + float(residual[t]))
 *   if residual:    residual[t] = s                    (in place; [T, H] bf16)
 *   out[t] = bf16(float(s) * rsqrt(mean(float(s)^2) + eps) * float(weight))
 * The sum of squares is taken in a fixed order (deterministic). residual may be null when
 * residual_in == 0 (plain RMSNorm). out must not alias x or residual. Requires H % 8 == 0,
 * 8 <= H <= 16384, 1 <= top_k <= 64.
 */
int tsm_add_rmsnorm(const void* x, int64_t T, int H, int top_k, void* residual, int residual_in,
                    const void* weight, float eps, void* out, hipStream_t stream);

/*
 * ---- Attention side of the qwen3_moe decoder (the end-to-end driver's own kernels) ----
 *
 * KV cache: K pages [num_pages, page, Hkv, D] bf16 (the reference's layout); V pages stored
 * transposed, [num_pages, Hkv, D, page] bf16 (so both MFMA operands of P.V read contiguous
 * memory). A cache slot is page_index * page + offset.
 *
 * In place on q [T, H, D] and k [T, Hkv, D] (strided rows, unit stride within a head): optional
 * per-head RMSNorm (q_weight / k_weight [D] bf16, both or neither; rounded to bf16), then
 * rotate-half RoPE with cos / sin [T, D/2] fp32 (row stride cs_stride):
 *   [x1, x2] -> [bf16(x1 cos - x2 sin), bf16(x2 cos + x1 sin)]
 * With k_cache given, also writes the rotated k and v [T, Hkv, D] into the cache (num_pages
 * pages of `page` slots) at slot_mapping[t] (int64; negative or past the pool: not written).
 * Replaces qk_norm_rope / _qk_norm_rope_kernel (tinykernels.py:107-275) and serve.py's
 * index_copy_ of K/V into the page pool (serve.py:898-904). Requires D even, D <= 128.
 */
int tsm_qk_norm_rope(void* q, int64_t T, int H, int64_t q_tok_stride, int64_t q_head_stride,
                     void* k, int Hkv, int64_t k_tok_stride, int64_t k_head_stride,
                     const void* v, int64_t v_tok_stride, int64_t v_head_stride, int D,
                     const float* cos, const float* sin, int64_t cs_stride,
                     const void* q_weight, const void* k_weight, float eps, void* k_cache,
                     void* v_cache, int64_t num_pages, int page, const int64_t* slot_mapping,
                     hipStream_t stream);

/*
 * Paged causal attention over packed requests: request b owns query rows
 * [query_start_loc[b], query_start_loc[b+1]) of q [T, H, D] and a context of
 * cu_seqlens_k[b+1] - cu_seqlens_k[b] tokens whose pages are block_table[b, :]; its queries are
 * the last q_len positions of that context, each attending to keys at positions <= its own.
 * GQA: query head h reads KV head h / (H / Hkv). out [T, H, D] bf16 (strided like q).
 * Block-table entries are clamped into [0, num_pages) (metadata is trusted, as in the
 * reference, but a wrong entry cannot address memory outside the caches).
 * Requests with one query token run in one launch (each workgroup's four wavefronts split the
 * context), longer ones in a second (skipped when max_query_len <= 1); the grids depend on T,
 * num_seqs, Hkv and num_splits only, so a step can be captured in a HIP graph.
 * Split-KV (num_splits > 1, at most 64): the one-token requests' contexts are cut into
 * num_splits contiguous ranges of 32-key blocks, one workgroup each, whose normalised partial
 * outputs and log-sum-exps go to `ws` (tsm_paged_attention_workspace_size bytes, 256-byte
 * aligned; unused with one split) and are merged in split order by a second launch, as the
 * reference's split-KV decode (_num_splits / _combine_splits_kernel, tinykernels.py:801-889).
 * Replaces paged_attention / _paged_attn_kernel (tinykernels.py:309-1028); results are those
 * of torch_ref_attention (serve.py:639-688). Requires D in {64, 128}, H / Hkv dividing 16,
 * page % 4 == 0, 16-byte aligned q rows.
 */
size_t tsm_paged_attention_workspace_size(int num_seqs, int H, int D, int num_splits);
int tsm_paged_attention(const void* q, int64_t T, int H, int64_t q_tok_stride,
                        int64_t q_head_stride, const void* k_cache, const void* v_cache,
                        int64_t num_pages, int page, int Hkv, int D, const int32_t* query_start_loc,
                        const int32_t* cu_seqlens_k, const int32_t* block_table,
                        int64_t bt_stride, int num_seqs, int max_query_len, float scale,
                        int num_splits, void* ws, size_t ws_bytes, void* out,
                        int64_t o_tok_stride, int64_t o_head_stride, hipStream_t stream);

/*
 * Greedy token choice: out[r] = the index of the largest of logits[r, 0..V) (row stride ld,
 * dtype TSM_F32 or TSM_BF16), the lowest index among equal values (torch.argmax's first
 * maximal index; serve.py's greedy path, temperature 0).
 */
int tsm_greedy_argmax(const void* logits, int dtype, int64_t rows, int64_t ld, int V,
                      int64_t* out, hipStream_t stream);

/*
 * MFMA-tiled ("packed") expert weights. No counterpart in the reference, which streams w13/w2 in
 * their checkpoint layout (tinykernels.py:1707-1738); this is a one-time reordering (same size)
 * after which every 16x16x32 MFMA operand of a 16-row block is 1 KiB of contiguous memory:
 *   packed[e][blk][s][lane][i] = W[e][16*src(blk) + lane%16][32*s + 8*(lane/16) + i]
 * with src(blk) = blk for w2 ([E, H, I]: N = H, K = I, interleave_halves = 0) and, for w13
 * ([E, 2I, H]: N = 2I, K = H, interleave_halves = 1), src(2j) = j, src(2j+1) = I/16 + j (gate
 * block j next to its up block). Requires N % 16 == 0 (N % 32 with interleaving), K % 32 == 0.
 * The *_packed entry points are tsm_fused_moe / tsm_moe_forward on packed weights.
 */
int tsm_moe_pack_weights(const void* w, int64_t E, int N, int K, int interleave_halves, void* out,
                         hipStream_t stream);
/*
 * Packing with zero padding, for shapes the tile kernels do not take as they are (the reference's
 * _fused_moe_kernel masks a ragged last K/N block instead, tinykernels.py:1719-1731; e.g. the
 * one-GPU share of TP-8 for Qwen3-30B-A3B has I = 768/8 = 96). The source is [E, N, K]
 * (interleave_halves: N = 2I, gate rows then up rows); the output is [E, N_pad, K_pad] in the
 * packed layout above, with W read as zero outside the source. A padded row or column adds exact
 * zeros to every product and sum, so outputs equal those of the unpadded problem.
 * tsm_moe_padded_shape gives the sizes the *_packed entry points run at: H_pad = H and
 * I_pad = I when the kernels take them, else H rounded up to a multiple of 128 and I to a
 * multiple of 128. Pack w13 with (N, K, N_pad, K_pad) = (2I, H, 2 I_pad, H_pad) and w2 with
 * (H, I, H_pad, I_pad); the *_packed entry points are then called with H = H_pad and I = I_pad,
 * and x / out carry H_pad columns (x zero-padded; the extra output columns are zero).
 */
int tsm_moe_padded_shape(int H, int I, int* H_pad, int* I_pad);
int tsm_moe_pack_weights_padded(const void* w, int64_t E, int N, int K, int N_pad, int K_pad,
                                int interleave_halves, void* out, hipStream_t stream);
int tsm_fused_moe_packed(const void* x, const void* w13p, const void* w2p, const float* topk_w,
                         const int32_t* topk_ids, int64_t T, int H, int I, int E, int top_k,
                         int sum_topk, void* out, void* ws, size_t ws_bytes, hipStream_t stream);
int tsm_moe_forward_packed(const void* x, const void* gate_w, const void* w13p, const void* w2p,
                           const int64_t* expert_map, const float* bias, int64_t T, int H, int I,
                           int E, int top_k, int renorm, int logits_bf16, int sum_topk, void* out,
                           float* topk_w, int32_t* topk_ids, void* ws, size_t ws_bytes,
                           hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* TINYSERVE_MOE_H */
