"""The MoE functions of tinyserve's `tinykernels` module, same names and call signatures, running
the gfx950 HIP kernels. `SparseMoE.forward` (serve.py:1076-1087) calls these through
`import tinykernels as tk`; pointing that import here is the drop-in.

    moe_route(logits, top_k, renormalize, expert_map)          tinykernels.py:1573
    moe_align_block_size(topk_ids, block_m, num_experts)       tinykernels.py:1070
    moe_align_block_size_triton(topk_ids, block_m, num_experts) tinykernels.py:1462
    silu_and_mul(gate, up)                                     tinykernels.py:299
    fused_moe(x, w13, w2, topk_weights, topk_ids, sum_topk)    tinykernels.py:1767
    autotune_fused_moe(w13, w2, top_k, max_num_tokens)         tinykernels.py:1799
"""
import torch

from . import ops
from ._lib import lib


def moe_route(logits: torch.Tensor, top_k: int, renormalize: bool, expert_map: torch.Tensor):
    """logits [T, E] -> topk_weights fp32 [T, top_k], topk_ids int32 [T, top_k] (local ids)."""
    return ops.moe_route(logits, top_k, renormalize, expert_map)


def moe_align_block_size(topk_ids: torch.Tensor, block_m: int, num_experts: int):
    return ops.moe_align_block_size(topk_ids, block_m, num_experts)


# The reference has a torch and a Triton version with identical outputs; both names map here.
moe_align_block_size_triton = moe_align_block_size


def silu_and_mul(gate: torch.Tensor, up: torch.Tensor):
    return ops.silu_and_mul(gate, up)


def fused_moe(x, w13, w2, topk_weights, topk_ids, sum_topk=True):
    """x [T, H], w13 [E, 2I, H] (gate rows then up rows), w2 [E, H, I], topk_weights/topk_ids
    [T, top_k] (ids local, -1 = another GPU's). Returns sum_k weight_k * expert_k(x) as [T, H]
    (or the [T*top_k, H] per-slot rows when sum_topk is False)."""
    return ops.fused_moe(x, w13, w2, topk_weights, topk_ids, sum_topk)


def moe_block_m(T: int, H: int, I: int, E: int, top_k: int, packed: bool = False) -> int:
    """Tile height fused_moe (packed=False) or fused_moe_packed (packed=True) uses for T tokens
    (its own table, not the reference's rule)."""
    return int(lib.tsm_moe_block_m(T, H, I, E, top_k, int(packed)))


@torch.inference_mode()
def autotune_fused_moe(w13: torch.Tensor, w2: torch.Tensor, top_k: int, max_num_tokens: int):
    """The kernel choice is a static table, so there is nothing to tune: this warms the code objects
    up for the same two batch sizes the reference tunes at (1 and max_num_tokens)."""
    E, H = w13.shape[0], w13.shape[2]
    for T in (1, max_num_tokens):
        x = torch.randn(T, H, device=w13.device, dtype=w13.dtype)
        ids = torch.randint(0, E, (T, top_k), device=w13.device)
        weights = torch.rand(T, top_k, device=w13.device)
        fused_moe(x, w13, w2, weights, ids)
