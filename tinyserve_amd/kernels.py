"""The MoE functions of tinyserve's `tinykernels` module, same names and call signatures, running
the gfx950 HIP kernels. `SparseMoE.forward` (serve.py:1076-1087) calls these through
`import tinykernels as tk`; pointing that import here is the drop-in.

    moe_route(logits, top_k, renormalize, expert_map)          tinykernels.py:1573
    moe_align_block_size(topk_ids, block_m, num_experts)       tinykernels.py:1070
    moe_align_block_size_triton(topk_ids, block_m, num_experts) tinykernels.py:1462
    silu_and_mul(gate, up)                                     tinykernels.py:299
    fused_moe(x, w13, w2, topk_weights, topk_ids, sum_topk)    tinykernels.py:1767
    autotune_fused_moe(w13, w2, top_k, max_num_tokens)         tinykernels.py:1799

autotune_fused_moe times the kernel families and tile heights this build has (expert-major,
16-, 64- and, with packed weights, 128- and 256-row tiles) per power-of-two bucket of assignment
counts and installs the fastest in the library's plan table (set_moe_block_m). 256-row tiles
exist only through it: the static table never picks them.
"""
import warnings

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


def set_moe_block_m(numel_lo: int, numel_hi: int, block_m: int, packed: bool = False):
    """Install a tile height for assignment counts in [numel_lo, numel_hi] (their power-of-two
    buckets); block_m = -1 restores the static table (tsm_moe_set_block_m)."""
    from ._lib import check
    check(lib.tsm_moe_set_block_m(numel_lo, numel_hi, int(packed), block_m), "set_moe_block_m")


def _agrees(out: torch.Tensor, ref: torch.Tensor) -> bool:
    """Two plans' results of one layer agree: finite, and within the bf16 layer tolerance
    (max-abs 2e-2 and mean relative 5e-3, relative to the result's own scale)."""
    if not bool(torch.isfinite(out).all()):
        return False
    d = (out.float() - ref.float()).abs()
    scale = ref.float().abs()
    return (d.max().item() <= 2e-2 * max(1.0, scale.max().item())
            and d.mean().item() <= 5e-3 * max(scale.mean().item(), 1e-30))


def _candidates(numel: int, E: int, packed: bool):
    c = [16, 64] + ([128] if packed else [])
    if packed and numel > 32 * E:   # 256-row tiles: only where experts average > 32 rows
        c.append(256)
    if numel <= 4096:   # the expert-major stages' row limit
        c.insert(0, 0)
    return c


@torch.inference_mode()
def autotune_fused_moe(w13: torch.Tensor, w2: torch.Tensor, top_k: int, max_num_tokens: int,
                       packed: bool = False, reps: int = 5):
    """Time the tile heights fused_moe can run for batch sizes 1, 2, 4, ... up to
    max_num_tokens (random routing on the real expert weights, as the reference tunes,
    tinykernels.py:1798-1811) and install the fastest for each power-of-two bucket of
    assignment counts. `packed`: w13/w2 are pack_moe_weights output and the packed-layout plans
    are tuned. Every candidate's output is first checked against the static plan's on the same
    input; a plan that disagrees (beyond the bf16 tolerance of a layer) is never installed, and
    a warning names it. Returns {numel bucket start: (block_m, microseconds)}."""
    fn = ops.fused_moe_packed if packed else fused_moe
    E, H = w13.shape[0], w13.shape[2]
    dev = w13.device
    table = {}
    T = 1
    sizes = []
    while T < max_num_tokens:
        sizes.append(T)
        T *= 2
    sizes.append(max_num_tokens)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for T in sizes:
        numel = T * top_k
        x = torch.randn(T, H, device=dev, dtype=torch.bfloat16)
        ids = torch.randint(0, E, (T, top_k), device=dev, dtype=torch.int32)
        weights = torch.rand(T, top_k, device=dev)
        best = None
        set_moe_block_m(numel, numel, -1, packed)
        ref = fn(x, w13, w2, weights, ids)   # the static plan's result: what tuning must keep
        for bm in _candidates(numel, E, packed):
            set_moe_block_m(numel, numel, bm, packed)
            if moe_block_m(T, H, w2.shape[-1], E, top_k, packed) != bm:
                continue   # the shape has no kernel at this height
            out = fn(x, w13, w2, weights, ids)  # warm-up, and the check
            if not _agrees(out, ref):
                warnings.warn(f"autotune_fused_moe: the {bm}-row plan disagrees with the static "
                              f"plan at T={T}; not installed")
                continue
            start.record()
            for _ in range(reps):
                fn(x, w13, w2, weights, ids)
            stop.record()
            stop.synchronize()
            us = start.elapsed_time(stop) * 1e3 / reps
            if best is None or us < best[1]:
                best = (bm, us)
        set_moe_block_m(numel, numel, best[0] if best else -1, packed)
        if best:
            table[1 << (numel.bit_length() - 1)] = best
    return table
