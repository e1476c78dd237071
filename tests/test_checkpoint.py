"""Checkpoint layout adapter (CPU): per-expert safetensors tensors land in the stacked w13 / w2
rows the reference's load_expert defines (serve.py:1052-1074), the router weight in gate, and
experts outside an expert-parallel block's range are skipped."""
from types import SimpleNamespace

import torch
from safetensors.torch import save_file

from tinyserve_amd.checkpoint import load_moe_checkpoint, missing_moe_weights
from tinyserve_amd.moe import SparseMoE

E, H, I = 8, 64, 32


def cfg(local=None):
    c = SimpleNamespace(num_experts=E, hidden_size=H, moe_intermediate_size=I,
                        num_experts_per_tok=2, norm_topk_prob=True)
    if local is not None:
        c.local_experts = local
    return c


def test_load_moe_checkpoint(tmp_path):
    g = torch.Generator().manual_seed(0)
    tensors = {}
    for L in (0, 3, 5):
        pre = "model." if L != 3 else ""  # both key spellings occur in checkpoints
        tensors[f"{pre}layers.{L}.mlp.gate.weight"] = torch.randn(E, H, generator=g)
        for e in range(E):
            for proj, shape in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
                tensors[f"{pre}layers.{L}.mlp.experts.{e}.{proj}.weight"] = torch.randn(
                    *shape, generator=g)
    tensors["model.layers.0.self_attn.q_proj.weight"] = torch.randn(4, 4, generator=g)
    keys = sorted(tensors)
    a, b = tmp_path / "a.safetensors", tmp_path / "b.safetensors"
    save_file({k: tensors[k] for k in keys[::2]}, str(a))   # experts split across files
    save_file({k: tensors[k] for k in keys[1::2]}, str(b))

    full, ep = SparseMoE(cfg()), SparseMoE(cfg(local=(2, 4)))
    loaded = load_moe_checkpoint({0: full, 3: ep}, [str(a), str(b)])

    assert missing_moe_weights(full, loaded[0]) == set()
    for e in range(E):
        p = f"model.layers.0.mlp.experts.{e}"
        assert torch.equal(full.w13[e, :I], tensors[f"{p}.gate_proj.weight"])
        assert torch.equal(full.w13[e, I:], tensors[f"{p}.up_proj.weight"])
        assert torch.equal(full.w2[e], tensors[f"{p}.down_proj.weight"])
    assert torch.equal(full.gate.weight, tensors["model.layers.0.mlp.gate.weight"])

    # expert parallel block: experts 2..5 only, stored at local slots 0..3
    assert missing_moe_weights(ep, loaded[3]) == set()
    assert not any(f":{e}:" in k for k in loaded[3] for e in (0, 1, 6, 7))
    for e in range(2, 6):
        p = f"layers.3.mlp.experts.{e}"
        assert torch.equal(ep.w13[e - 2, :I], tensors[f"{p}.gate_proj.weight"])
        assert torch.equal(ep.w2[e - 2], tensors[f"{p}.down_proj.weight"])
    assert 5 not in loaded  # layers without a block are ignored


def test_missing_reported():
    m = SparseMoE(cfg())
    miss = missing_moe_weights(m, {"gate", "w13:0:gate_proj"})
    assert "w13:0:up_proj" in miss and "w2:7:down_proj" in miss and "gate" not in miss
