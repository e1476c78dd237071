"""SparseMoE's in-place packed layout (no GPU: the HIP packing op is replaced by the tensor-
permutation statement of the same layout, tinyserve_amd.layout.pack, which test_layout pins).
The module keeps one copy of its expert weights, hands them back in the reference layout through
state_dict / unpack, restores the reference layout before loading, refuses to run on weights
written while packed, pads shapes the kernels do not take, and slices TP-MoE shards."""
from types import SimpleNamespace

import pytest
import torch

import tinyserve_amd
from tinyserve_amd import layout, ops
from tinyserve_amd import moe as moe_mod


@pytest.fixture
def counting_pack(monkeypatch):
    calls = []

    def fake_pack(w13, w2):
        calls.append(1)
        E, two_i, H = w13.shape
        Hp, Ip = ops.padded_shape(H, two_i // 2)
        return layout.pack(w13, True, 2 * Ip, Hp), layout.pack(w2, False, Hp, Ip)
    monkeypatch.setattr(moe_mod.ops, "pack_moe_weights", fake_pack)
    return calls


def make(E=4, H=128, I=64, **kw):
    cfg = SimpleNamespace(num_experts=E, hidden_size=H, moe_intermediate_size=I,
                          num_experts_per_tok=2, norm_topk_prob=True, **kw)
    m = tinyserve_amd.SparseMoE(cfg)
    g = torch.Generator().manual_seed(E * 100 + I)
    with torch.no_grad():
        m.w13.copy_(torch.randn(m.w13.shape, generator=g))
        m.w2.copy_(torch.randn(m.w2.shape, generator=g))
    return m


def test_pack_in_place_and_state_dict(counting_pack):
    m = make()
    w13, w2 = m.w13.detach().clone(), m.w2.detach().clone()
    m.pack()
    m.pack()
    assert len(counting_pack) == 1 and m.weights_packed
    assert torch.equal(m.w13, layout.pack(w13, True)) and torch.equal(m.w2, layout.pack(w2, False))
    # one copy: the parameters themselves hold the packed layout
    assert sorted(n for n, _ in m.named_parameters()) == ["gate.weight", "w13", "w2"]
    sd = m.state_dict()
    assert torch.equal(sd["w13"], w13) and torch.equal(sd["w2"], w2)
    m.unpack()
    assert not m.weights_packed and torch.equal(m.w13, w13) and torch.equal(m.w2, w2)


def test_writes_while_packed_are_refused(counting_pack):
    m = make()
    m.pack()
    with torch.no_grad():
        m.w13[1, :64].fill_(2.0)           # reference-layout write into packed storage
    with pytest.raises(RuntimeError, match="packed layout"):
        m.pack()


def test_load_state_dict_restores_reference_layout(counting_pack):
    src, dst = make(), make(E=4, I=64)
    dst.pack()
    dst.load_state_dict(src.state_dict())
    assert not dst.weights_packed
    assert torch.equal(dst.w13, src.w13) and torch.equal(dst.w2, src.w2)
    dst.pack()
    assert len(counting_pack) == 2 and torch.equal(dst.w13, layout.pack(src.w13.detach(), True))


def test_force_repack_after_data_write(counting_pack):
    m = make()
    m.pack()
    ref13, ref2 = torch.full((4, 128, 128), 3.0), torch.full((4, 128, 64), 5.0)
    m.w13.data.copy_(ref13)                # through .data: the version counter does not move
    m.w2.data.copy_(ref2)
    m.pack(force=True)
    assert torch.equal(m.state_dict()["w13"], ref13) and torch.equal(m.state_dict()["w2"], ref2)


def test_padded_shape_round_trip(counting_pack):
    """I = 24 (the kernels take I % 64 == 0): packed tensors carry the zero-padded size."""
    m = make(E=2, H=128, I=24)
    w13, w2 = m.w13.detach().clone(), m.w2.detach().clone()
    m.pack()
    assert tuple(m.w13.shape) == (2, 256, 128) and tuple(m.w2.shape) == (2, 128, 128)
    sd = m.state_dict()
    assert torch.equal(sd["w13"], w13) and torch.equal(sd["w2"], w2)
    m.unpack()
    assert tuple(m.w13.shape) == (2, 48, 128) and torch.equal(m.w13, w13)


class FakeSlice:
    def __init__(self, t):
        self.t = t

    def get_shape(self):
        return list(self.t.shape)

    def __getitem__(self, idx):
        return self.t[idx]


class FakeFile:
    def __init__(self, tensors):
        self.tensors = tensors

    def get_tensor(self, key):
        return self.tensors[key]

    def get_slice(self, key):
        return FakeSlice(self.tensors[key])


def test_tp_moe_load_slices(counting_pack):
    """TP-2 MoE: rank r holds rows [r I/2, (r+1) I/2) of gate_proj / up_proj and the same
    columns of down_proj (serve.py:731-777), into a module built at I/2."""
    H, I = 128, 64
    g = torch.Generator().manual_seed(7)
    full = {f"experts.0.{p}.weight": torch.randn(s, generator=g)
            for p, s in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I)))}
    fh = FakeFile(full)
    for rank in (0, 1):
        m = make(E=1, H=H, I=I // 2)
        m.pack()                       # loading restores the reference layout first
        for p in ("gate_proj", "up_proj", "down_proj"):
            assert m.load_expert(0, p, fh, f"experts.0.{p}.weight", rank=rank, tp=2)
        sl = slice(rank * I // 2, (rank + 1) * I // 2)
        assert torch.equal(m.w13[0, :I // 2], full["experts.0.gate_proj.weight"][sl])
        assert torch.equal(m.w13[0, I // 2:], full["experts.0.up_proj.weight"][sl])
        assert torch.equal(m.w2[0], full["experts.0.down_proj.weight"][:, sl])


def test_router_logits_mode():
    m = make()
    assert not m._logits_bf16()        # fp32 gate: the reference's Linear output is fp32 too
    m.gate.to(torch.bfloat16)
    assert m._logits_bf16()            # bf16 gate: logits rounded to bf16, as serve.py's Linear
    m.router_logits = "fp32"
    assert not m._logits_bf16()
    with pytest.raises(ValueError):
        tinyserve_amd.SparseMoE(SimpleNamespace(num_experts=4, hidden_size=128,
                                                moe_intermediate_size=64, num_experts_per_tok=2),
                                router_logits="bf17")
