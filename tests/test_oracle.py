"""CPU tests that pin the oracle itself (no GPU): known-answer examples from the reference's
docstrings, closed forms, brute force on tiny inputs and invariants, each chosen so that a plausible
mistake (dropped term, wrong index, transposed operand, unstable order) fails."""
import json
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import c_oracle
from oracle.moe_oracle import (make_layer, moe_align_block_size_np, moe_reference,
                               moe_rows_reference, per_token_fp64, route_torch)

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "docstring_examples.json")))


# ------------------------------------------------------------------ align
def test_align_docstring_example_both_oracles():
    ex = GOLD["align_example"]
    ids = np.array(ex["topk_ids"], np.int32)
    for s, e, t in (c_oracle.align(ids, ex["block_m"], ex["num_experts"]),
                    moe_align_block_size_np(ids, ex["block_m"], ex["num_experts"])):
        assert s.tolist() == ex["sorted_token_ids"]
        assert e.tolist() == ex["expert_ids"]
        assert t.tolist() == ex["num_post_padded"]
    mid = GOLD["align_intermediates"]
    s, e, t = c_oracle.align(ids, ex["block_m"], ex["num_experts"])
    for d, o in zip(mid["dest"], mid["order"]):          # sorted_ids[dest[i]] = order[i]
        assert s[d] == o
    for b, (st, en) in enumerate(zip(mid["padded_start"], mid["padded_end"])):
        assert all(e[r // ex["block_m"]] == (b if b < 3 else -1) for r in range(st, en, 4))


def test_gemm_row_lookup_example():
    ex = GOLD["gemm_row_lookup"]
    s = np.array(ex["sorted_token_ids_prefix"])
    offs = s[ex["rows"]]
    assert offs.tolist() == ex["offs_token"]
    assert (offs < ex["num_valid_tokens"]).tolist() == ex["token_mask"]


def brute_align(ids, bm, E):
    """Independent O(numel * E) construction straight from the definition."""
    flat = [int(v) if 0 <= v < E else E for v in np.asarray(ids).ravel()]
    numel = len(flat)
    rows, eids = [], []
    for b in range(E + 1):
        members = [a for a in range(numel) if flat[a] == b]
        padded = -(-len(members) // bm) * bm
        rows += members + [numel] * (padded - len(members))
        eids += [b if b < E else -1] * (padded // bm)
    total = len(rows)
    mp = -(-(numel + (E + 1) * (bm - 1)) // bm) * bm
    rows += [numel] * (mp - total)
    eids += [-1] * (mp // bm - len(eids))
    return np.array(rows, np.int32), np.array(eids, np.int32), np.array([total], np.int32)


@pytest.mark.parametrize("seed", range(12))
def test_align_oracles_vs_brute_force(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 9))
    bm = int(rng.choice([1, 2, 4, 16]))
    T, k = int(rng.integers(0, 20)), int(rng.integers(1, 4))
    ids = rng.integers(-1, E, size=(T, k)).astype(np.int32)
    want = brute_align(ids, bm, E)
    for got in (c_oracle.align(ids, bm, E), moe_align_block_size_np(ids, bm, E)):
        for g, w in zip(got, want):
            assert np.array_equal(g, w)


def test_align_invariants_large():
    rng = np.random.default_rng(7)
    E, bm = 128, 64
    ids = rng.integers(-1, E, size=(3000, 8)).astype(np.int32)
    s, e, t = c_oracle.align(ids, bm, E)
    numel = ids.size
    real = s[s < numel]
    assert np.array_equal(np.sort(real), np.arange(numel))        # a permutation
    flat = np.where(ids.ravel() < 0, E, ids.ravel())
    for b in (0, 17, E):
        pos = np.nonzero(np.isin(s, np.nonzero(flat == b)[0]))[0]
        assert np.all(np.diff(s[pos]) > 0)                        # stable inside a bucket
    counts = np.bincount(flat, minlength=E + 1)
    assert t[0] == int(np.sum(-(-counts // bm) * bm))
    used = e[: t[0] // bm]
    assert np.all(np.diff(used[used >= 0]) >= 0) and np.all(e[t[0] // bm:] == -1)


# ------------------------------------------------------------------ exp / router
def test_oracle_expf_accuracy():
    x = np.concatenate([np.linspace(-86, 0, 40001), -np.logspace(-8, 1.9, 2000), [0.0, -0.0]])
    x = x.astype(np.float32)
    got = c_oracle.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.abs(got - ref) / np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 1.0, ulp.max()
    assert c_oracle.expf(np.array([-np.inf, np.nan, -87.0]))[:3].tolist() == [0.0, 0.0, 0.0]
    assert c_oracle.expf(np.array([0.0]))[0] == 1.0


def bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_router_logits_vs_float64():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(6, 2048, generator=g).bfloat16()
    w = (torch.randn(16, 2048, generator=g) * 0.02).bfloat16()
    got = c_oracle.router_logits(bf16_bits(x), bf16_bits(w))
    ref = (x.double() @ w.double().t()).numpy()
    scale = (x.double().abs() @ w.double().abs().t()).numpy()
    assert np.all(np.abs(got - ref) <= 2e-6 * scale + 1e-30)
    # fp32 inputs and a ragged H that leaves lanes empty
    x32 = torch.randn(3, 136, generator=g)
    w32 = torch.randn(5, 136, generator=g)
    got = c_oracle.router_logits(x32.numpy(), w32.numpy(), bias=np.arange(5, dtype=np.float32))
    ref = (x32.double() @ w32.double().t()).numpy() + np.arange(5)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_router_logits_bf16_mode_is_torch_rounding():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 512, generator=g).bfloat16()
    w = torch.randn(8, 512, generator=g).bfloat16()
    l32 = c_oracle.router_logits(bf16_bits(x), bf16_bits(w))
    l16 = c_oracle.router_logits(bf16_bits(x), bf16_bits(w), logits_bf16=True)
    assert np.array_equal(l16, torch.from_numpy(l32).bfloat16().float().numpy())


@pytest.mark.parametrize("renorm", [True, False])
def test_route_vs_closed_form(renorm):
    """ids = stable descending sort of p (lowest index first on ties); weights = torch's
    softmax -> top-k -> renormalise of serve.py:1089-1096 to fp32 rounding."""
    g = torch.Generator().manual_seed(2)
    logits = (torch.randn(300, 128, generator=g) * 3).bfloat16().float()  # many exact ties
    w, ids = c_oracle.route(logits.numpy(), 8, renorm)
    p = logits.numpy() - logits.numpy().max(1, keepdims=True)
    p = np.stack([c_oracle.expf(r) for r in p])
    order = np.argsort(-p, axis=1, kind="stable")[:, :8]
    assert np.array_equal(ids, order)
    tw, tids = route_torch(logits, 8, renorm)
    assert np.allclose(w, tw.numpy(), rtol=3e-6, atol=1e-8)
    if renorm:
        assert np.allclose(w.sum(1), 1.0, atol=2e-6)
    assert np.all(np.diff(w, axis=1) <= 0)


def test_route_ties_brute_force():
    logits = np.zeros((3, 8), np.float32)
    logits[1] = [1, 3, 3, 0, 3, 2, 2, 1]
    logits[2] = [-np.inf] * 4 + [0, 0, 1, 1]
    w, ids = c_oracle.route(logits, 3, True)
    assert ids.tolist() == [[0, 1, 2], [1, 2, 4], [6, 7, 4]]
    assert np.allclose(w[0], 1 / 3) and np.allclose(w[1], 1 / 3)
    emap = np.array([3, 2, 1, 0, -1, -1, 7, 6], np.int64)
    _, mids = c_oracle.route(logits, 3, True, emap)
    assert mids.tolist() == [[3, 2, 1], [2, 1, -1], [7, 6, -1]]


def test_route_non_renorm_denominator_is_sum_of_all():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(50, 60, generator=g)
    w, ids = c_oracle.route(logits.numpy(), 4, False)
    probs = logits.double().softmax(-1).numpy()
    assert np.allclose(w, np.take_along_axis(probs, ids.astype(np.int64), 1), rtol=2e-6)


# ------------------------------------------------------------------ experts
def test_routing_example_nonzero():
    ex = GOLD["routing_example"]
    ids = torch.tensor(ex["topk_ids"])
    tok, slot = (ids == ex["expert"]).nonzero(as_tuple=True)
    assert tok.tolist() == ex["tok"] and slot.tolist() == ex["slot"]


def test_moe_reference_vs_fp64_textbook():
    """Pins gate-vs-up order, silu placement, weight application and the down transpose."""
    x, gw, w13, w2 = make_layer(64, 256, 8, 512, torch.float32, seed=0)
    w, ids = route_torch(x @ gw.t(), 2, True)
    out = moe_reference(x, w13, w2, w, ids)
    ref = per_token_fp64(x, w13, w2, w, ids)
    assert torch.allclose(out.double(), ref, rtol=1e-4, atol=1e-5)
    # a swapped gate/up order would not pass
    swapped = torch.cat([w13[:, 512:], w13[:, :512]], 1)
    assert not torch.allclose(moe_reference(x, swapped, w2, w, ids).double(), ref, atol=1e-3)


def test_moe_reference_remote_ids_contribute_zero():
    x, gw, w13, w2 = make_layer(16, 256, 8, 512, torch.float32, seed=1)
    w, ids = route_torch(x @ gw.t(), 2, True)
    ids_remote = torch.where(ids >= 4, torch.full_like(ids, -1), ids)
    out = moe_reference(x, w13, w2, w, ids_remote)
    ref = per_token_fp64(x, w13, w2, w, ids_remote)
    assert torch.allclose(out.double(), ref, rtol=1e-4, atol=1e-5)


def test_rows_reference_sums_to_reference():
    x, gw, w13, w2 = make_layer(32, 256, 8, 512, torch.float32, seed=2)
    w, ids = route_torch(x @ gw.t(), 2, True)
    rows = moe_rows_reference(x, w13, w2, w, ids)
    assert torch.allclose(rows.view(32, 2, 256).sum(1), moe_reference(x, w13, w2, w, ids),
                          atol=1e-5)


def test_bf16_rounding_points_of_reference():
    """In bf16 the reference rounds gate/up and silu to bf16 before the multiply."""
    x, gw, w13, w2 = make_layer(8, 256, 8, 512, torch.bfloat16, seed=3)
    ids = torch.tensor([[e, (e + 1) % 8] for e in range(8)])
    w = torch.full((8, 2), 0.5)
    out = moe_reference(x, w13, w2, w, ids)
    ref = per_token_fp64(x.float(), w13.float(), w2.float(), w, ids)
    err = (out.double() - ref).abs()
    assert err.max() < 2e-2 and (err.mean() / ref.abs().mean()) < 5e-3
    gu = x[:1] @ w13[0].t()
    assert torch.equal(F.silu(gu[:, :512]), F.silu(gu[:, :512].float()).bfloat16())


# ---------------------------------------------------------------- residual-add RMSNorm
def _bf16_ulp(v):
    return torch.exp2(torch.floor(torch.log2(v.abs().clamp_min(2.0 ** -126))) - 7)


@pytest.mark.parametrize("k,with_res", [(1, False), (1, True), (8, True), (2, False)])
def test_add_rmsnorm_reference_against_fp64(k, with_res):
    from oracle.moe_oracle import add_rmsnorm_reference
    g = torch.Generator().manual_seed(k * 10 + with_res)
    T, H, eps = 7, 256, 1e-6
    rows = (torch.randn(T * k, H, generator=g) * 0.5).bfloat16()
    res = (torch.randn(T, H, generator=g) * 2).bfloat16() if with_res else None
    w = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    out, new_res = add_rmsnorm_reference(rows, k, res, w, eps)
    # the k-sum: float64 sum rounded to bf16, within one rounding of it
    s64 = rows.double().view(T, k, H).sum(1)
    x = s64.to(torch.bfloat16)
    assert bool(((new_res.double() - (x.double() if res is None else
                                      (x.double() + res.double()))).abs()
                 <= _bf16_ulp(new_res.double()) * (1 if res is None else 2)).all())
    if res is not None and k == 1:   # one bf16 rounding of the fp32 sum of the two bf16 inputs
        assert torch.equal(new_res, (rows.float() + res.float()).bfloat16())
    r = new_res.double()
    ref = r / torch.sqrt((r * r).mean(-1, keepdim=True) + eps) * w.double()
    assert bool(((out.double() - ref).abs() <= _bf16_ulp(ref) + 1e-30).all())


def test_add_rmsnorm_reference_known_answers():
    from oracle.moe_oracle import add_rmsnorm_reference
    H = 64
    w = torch.linspace(0.5, 2.0, H).bfloat16()
    rows = torch.full((3, H), -4.0).bfloat16()          # constant row: x / rms(x) = sign(x)
    out, res = add_rmsnorm_reference(rows, 1, None, w, 0.0)
    assert torch.equal(out, (-w.float()).bfloat16().expand(3, H))
    assert torch.equal(res, rows)
    # rows of two slots that cancel, plus a residual of ones: the norm sees the residual alone
    rows2 = torch.stack([torch.full((H,), 3.0), torch.full((H,), -3.0)]).bfloat16()
    out, res = add_rmsnorm_reference(rows2, 2, torch.ones(1, H).bfloat16(), w, 0.0)
    assert torch.equal(res, torch.ones(1, H).bfloat16()) and torch.equal(out[0], w)


def test_silu_and_mul_reference():
    from oracle.moe_oracle import silu_and_mul_reference
    g = torch.tensor([0.0, 20.0, -20.0, 1.0, -1.0]).bfloat16()
    u = torch.tensor([5.0, 2.0, 3.0, 1.0, 1.0]).bfloat16()
    out = silu_and_mul_reference(g, u).double()
    assert out[0] == 0 and abs(out[1] - 40.0) <= 0.25 and abs(out[2]) < 1e-6
    x = torch.randn(1000, generator=torch.Generator().manual_seed(0)).bfloat16() * 4
    y = torch.randn(1000, generator=torch.Generator().manual_seed(1)).bfloat16()
    ref = x.double() / (1 + torch.exp(-x.double())) * y.double()
    got = silu_and_mul_reference(x, y).double()
    # two roundings to bf16 (silu, then the product): within 2^-7 relative
    assert bool(((got - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-30).all())
