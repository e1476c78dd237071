"""Checkpoint layout adapter: per-expert safetensors tensors -> the stacked SparseMoE weights.

A qwen3_moe checkpoint stores every expert projection as its own tensor,
`[model.]layers.{L}.mlp.experts.{e}.{gate_proj|up_proj|down_proj}.weight`, plus the router
`[model.]layers.{L}.mlp.gate.weight`. The reference's loader routes the expert tensors to
`SparseMoE.load_expert` (serve.py:1338-1346, key pattern serve.py:71) and the router through its
generic parameter path. This module does the same for a set of SparseMoE blocks, file by file,
reading each tensor once through safetensors' memory-mapped `safe_open` (no unpickling), and
reports which weights of which layer were filled, so a caller can check that nothing is missing.
After loading, the modules repack their MFMA-tiled copies on their next forward (or at `pack()`).
"""
import re
from typing import Dict, Iterable, Mapping, Set

import torch

# The checkpoint key format of per-expert weights (the same pattern as serve.py:71: it is the
# file format being read, not an implementation choice).
EXPERT_KEY = re.compile(r"layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)\.weight")
ROUTER_KEY = re.compile(r"layers\.(\d+)\.mlp\.gate\.weight")


def load_moe_checkpoint(layers: Mapping[int, torch.nn.Module], paths: Iterable[str],
                        device: str = "cpu") -> Dict[int, Set[str]]:
    """Fill the SparseMoE blocks `layers[L]` from the safetensors files `paths`.

    Returns {layer: {"gate", "w13:<expert>:gate_proj", ...}} of what was loaded; experts outside
    a block's local range (expert parallelism) are skipped without being read. Keys of layers
    not in `layers`, and non-MoE keys, are ignored.
    """
    from safetensors import safe_open

    loaded: Dict[int, Set[str]] = {L: set() for L in layers}
    for path in paths:
        with safe_open(path, framework="pt", device=device) as fh:
            for key in fh.keys():
                name = key.removeprefix("model.")
                if m := EXPERT_KEY.fullmatch(name):
                    L = int(m[1])
                    if L in layers and layers[L].load_expert(int(m[2]), m[3], fh, key):
                        loaded[L].add(f"{'w2' if m[3] == 'down_proj' else 'w13'}:{m[2]}:{m[3]}")
                elif m := ROUTER_KEY.fullmatch(name):
                    L = int(m[1])
                    if L in layers:
                        with torch.no_grad():
                            layers[L].gate.weight.copy_(fh.get_tensor(key))
                        loaded[L].add("gate")
    return loaded


def missing_moe_weights(module: torch.nn.Module, loaded: Set[str]) -> Set[str]:
    """What `load_moe_checkpoint` did not fill for one block (empty when complete)."""
    want = {"gate"}
    for e in range(module.first_expert, module.first_expert + module.num_local):
        want |= {f"w13:{e}:gate_proj", f"w13:{e}:up_proj", f"w2:{e}:down_proj"}
    return want - loaded
