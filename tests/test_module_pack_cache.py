"""SparseMoE's packed-weight cache (no GPU: the packing op is replaced by a counting stand-in).
The MFMA-tiled copies are rebuilt after in-place changes to w13/w2 (version counters), after the
parameters are replaced, and on pack(force=True); not otherwise."""
from types import SimpleNamespace

import torch

import tinyserve_amd
from tinyserve_amd import moe as moe_mod


def test_pack_cache_invalidation(monkeypatch):
    calls = []

    def fake_pack(w13, w2):
        calls.append(1)
        return w13.detach().clone(), w2.detach().clone()
    monkeypatch.setattr(moe_mod.ops, "pack_moe_weights", fake_pack)
    cfg = SimpleNamespace(num_experts=4, hidden_size=128, moe_intermediate_size=64,
                          num_experts_per_tok=2, norm_topk_prob=True)
    m = tinyserve_amd.SparseMoE(cfg)
    with torch.no_grad():
        m.w13.zero_()
        m.w2.zero_()
    m.pack()
    m.pack()
    assert len(calls) == 1
    with torch.no_grad():
        m.w13[1, :64].fill_(2.0)           # in place through a view: repack
    a13, _ = m.pack()
    assert len(calls) == 2 and float(a13[1, 0, 0]) == 2.0
    m.w2.data.fill_(3.0)                   # through .data: not seen ...
    m.pack()
    assert len(calls) == 2
    _, a2 = m.pack(force=True)             # ... until forced
    assert len(calls) == 3 and float(a2[0, 0, 0]) == 3.0
    m.w13 = torch.nn.Parameter(torch.ones_like(m.w13))   # replaced parameter: repack
    m.pack()
    assert len(calls) == 4
