"""The product's kernels executed on the CPU (tests/emu: the HIP sources compiled as host C++
against a fiber-per-thread device stand-in) through the product's own Python ops, against the
oracles, at small sizes.

What this pins: the kernels' indexing, data movement, masking, plans, padding and orchestration
(the CPU build runs the same source); bit-exact where the arithmetic is exactly specified
(routing, the permutation, the fixed-order router, residual streams, packing). What it does not:
the GPU's own arithmetic (the matrix-core instruction is evaluated in double precision here) and
anything about timing, memory ordering between workgroups or the compiler's device code
generation. The -m gpu tests remain the parity tests proper.

The same cases also run under AddressSanitizer and ThreadSanitizer (test_emu_sanitizers.py), so
that an out-of-bounds access, or a data race between wavefronts or workgroups, of a kernel is
caught on the CPU."""
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "emu"))
sys.path.insert(0, HERE)

import harness  # noqa: E402
from oracle import c_oracle  # noqa: E402
from oracle.moe_oracle import (add_rmsnorm_reference, make_layer,  # noqa: E402
                               moe_align_block_size_np, moe_reference)

@pytest.fixture(scope="module")
def tsm():
    import tinyserve_amd
    with harness.emulated(harness.sanitizer_from_env()):
        yield tinyserve_amd


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def close(out, ref, max_abs=2e-2, mean_rel=5e-3):
    out, ref = out.float(), ref.float()
    assert torch.isfinite(out).all()
    assert (out - ref).abs().max().item() <= max_abs
    assert ((out - ref).abs().mean() / ref.abs().mean()).item() <= mean_rel


@pytest.mark.parametrize("T,E,k", [(1, 128, 8), (33, 60, 4), (7, 512, 8), (64, 8, 2)])
def test_route_bitexact(tsm, T, E, k):
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g) * 2
    logits[0, ::3] = 1.0                                 # ties
    w, ids = tsm.moe_route(logits, k, True, None)
    ow, oids = c_oracle.route(logits.numpy(), k, True)
    assert np.array_equal(ids.numpy(), oids) and same_bits(w.numpy(), ow)


@pytest.mark.parametrize("T", [3, 64, 300])
def test_router_fused(tsm, T):
    """T <= 256: the fixed-order kernels, bit-exact with the C oracle; T > 256: the matrix-core
    router, its logits within the fp32 accumulation bound and its selection bit-exact."""
    x, gw, _, _ = make_layer(T, 256, 16, 64, torch.bfloat16, seed=T)
    w, ids, logits = tsm.moe_router(x, gw, 4, True)
    if T <= 256:
        ol = c_oracle.router_logits(bits(x), bits(gw))
        assert same_bits(logits.numpy(), ol)
    else:
        exact = x.double() @ gw.double().t()
        bound = (x.double().abs() @ gw.double().abs().t()) * 2.0 ** -17
        assert bool(((logits.double() - exact).abs() <= bound).all())
        ol = logits.numpy()
    ow, oids = c_oracle.route(ol, 4, True)
    assert np.array_equal(ids.numpy(), oids) and same_bits(w.numpy(), ow)


@pytest.mark.parametrize("numel,E,bm", [(0, 8, 16), (37, 8, 16), (300, 16, 64), (9000, 32, 64)])
def test_align_bitexact(tsm, numel, E, bm):
    g = torch.Generator().manual_seed(numel)
    ids = torch.randint(-1, E, (numel,), generator=g, dtype=torch.int32)
    s, e, t = tsm.moe_align_block_size(ids, bm, E)
    rs, re_, rt = moe_align_block_size_np(ids.numpy(), bm, E)
    assert np.array_equal(s.numpy(), rs) and np.array_equal(e.numpy(), re_)
    assert int(t[0]) == int(rt[0])


@pytest.mark.parametrize("T", [2, 40, 300, 700])   # 700: experts past 128 rows (256-row tiles
def test_experts_every_plan(tsm, T):                # with both halves active)
    """Every plan the static table or the tuner can pick (expert-major, 16-, 64-row tiles;
    128- and 256-row persistent tiles on packed weights), both weight layouts, against the
    oracle; the packed and reference-layout kernels of a plan agree bit for bit, and so do the
    64-, 128- and 256-row tile kernels (one fp32 chain per output in the same k order)."""
    from tinyserve_amd import kernels
    H, E, I, k = 256, 8, 512, 2
    x, gw, w13, w2 = make_layer(T, H, E, I, torch.bfloat16, seed=10 + T)
    w, ids, _ = tsm.moe_router(x, gw, k, True)
    ref = moe_reference(x, w13, w2, w, ids.long())
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    numel = T * k
    tiles = {}
    try:
        for bm in (0, 16, 64, 128, 256):
            for packed in (False, True):
                if bm >= 128 and not packed:
                    continue
                kernels.set_moe_block_m(numel, numel, bm, packed)
                if kernels.moe_block_m(T, H, I, E, k, packed) != bm:
                    continue
                out = (tsm.fused_moe_packed(x, p13, p2, w, ids) if packed
                       else tsm.fused_moe(x, w13, w2, w, ids))
                close(out, ref)
                if packed and bm >= 64:
                    tiles[bm] = out
                if packed and bm < 128:
                    kernels.set_moe_block_m(numel, numel, bm, False)
                    assert torch.equal(out, tsm.fused_moe(x, w13, w2, w, ids)), bm
        assert set(tiles) == {64, 128, 256}
        assert torch.equal(tiles[64], tiles[128]) and torch.equal(tiles[128], tiles[256])
    finally:
        kernels.set_moe_block_m(1, 1 << 30, -1, False)
        kernels.set_moe_block_m(1, 1 << 30, -1, True)


@pytest.mark.parametrize("packed", [False, True])
def test_autotune_small_layer(tsm, packed):
    """autotune_fused_moe's logic on the host clock: one installed plan per power-of-two bucket,
    each a height the shape has a kernel for (256-row tiles among the packed candidates), the
    installed plans keep parity with the oracle, and clearing restores the static table."""
    from tinyserve_amd import kernels
    H, E, I, k = 256, 8, 512, 2
    x, gw, w13, w2 = make_layer(8, H, E, I, torch.bfloat16, seed=6)
    a, b = tsm.pack_moe_weights(w13, w2) if packed else (w13, w2)
    before = {T: kernels.moe_block_m(T, H, I, E, k, packed) for T in (1, 40, 300)}
    try:
        table = kernels.autotune_fused_moe(a, b, k, 300, packed=packed, reps=1)
        assert set(table) == {1 << (n.bit_length() - 1) for n in (2, 4, 8, 16, 32, 64, 128, 256,
                                                                     512, 600)}
        for bucket, (bm, _) in table.items():
            assert bm in ((0, 16, 64, 128, 256) if packed else (0, 16, 64)), (bucket, bm)
        for T in (1, 40, 300):
            bm, _ = table[1 << ((T * k).bit_length() - 1)]
            assert kernels.moe_block_m(T, H, I, E, k, packed) == bm
            xs = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).bfloat16()
            w, ids, _ = tsm.moe_router(xs, gw, k, True)
            fn = tsm.fused_moe_packed if packed else tsm.fused_moe
            close(fn(xs, a, b, w, ids), moe_reference(xs, w13, w2, w, ids.long()))
    finally:
        kernels.set_moe_block_m(1, 1 << 30, -1, packed)
    assert {T: kernels.moe_block_m(T, H, I, E, k, packed) for T in (1, 40, 300)} == before


def test_autotune_never_installs_a_disagreeing_plan(tsm, monkeypatch):
    """A plan whose results disagree with the static plan's (here the 16-row plan, made wrong
    on purpose on the host) is timed out of the table with a warning, whatever its speed."""
    from tinyserve_amd import kernels
    H, E, I, k = 256, 8, 512, 2
    _, _, w13, w2 = make_layer(8, H, E, I, torch.bfloat16, seed=6)
    real = kernels.fused_moe

    def wrong_at_16(x, w13_, w2_, w, ids, sum_topk=True):
        out = real(x, w13_, w2_, w, ids, sum_topk)
        if kernels.moe_block_m(x.shape[0], H, I, E, k, False) == 16:
            out = out + 1.0
        return out

    monkeypatch.setattr(kernels, "fused_moe", wrong_at_16)
    try:
        with pytest.warns(UserWarning, match="16-row plan disagrees"):
            table = kernels.autotune_fused_moe(w13, w2, k, 64, packed=False, reps=1)
        assert table and all(bm != 16 for bm, _ in table.values()), table
    finally:
        kernels.set_moe_block_m(1, 1 << 30, -1, False)


def test_expert_parallel_and_rows(tsm):
    H, E, I, k, T = 256, 16, 128, 4, 50
    x, gw, w13, w2 = make_layer(T, H, E, I, torch.bfloat16, seed=3)
    emap = torch.arange(E, dtype=torch.int64)
    emap[::2] = -1
    w, ids, _ = tsm.moe_router(x, gw, k, True, emap)
    assert bool((ids < 0).any())
    out = tsm.fused_moe(x, w13, w2, w, ids)
    close(out, moe_reference(x, w13, w2, w, ids.long()))
    rows = tsm.fused_moe(x, w13, w2, w, ids, sum_topk=False).view(T, k, H)
    assert bool((rows[ids < 0] == 0).all())
    assert torch.equal(rows.float().sum(1).bfloat16(), out)


def test_padded_shapes(tsm):
    """I = 96 (the TP-8 share of Qwen3-30B-A3B) and H = 200 through the zero-padded packing."""
    from tinyserve_amd import layout
    x, gw, w13, w2 = make_layer(40, 256, 16, 96, torch.bfloat16, seed=2)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    assert torch.equal(p13, layout.pack(w13, True, 256, 256))
    assert torch.equal(p2, layout.pack(w2, False, 256, 128))
    w, ids, _ = tsm.moe_router(x, gw, 4, True)
    out = tsm.fused_moe(x, w13, w2, w, ids)
    close(out, moe_reference(x, w13, w2, w, ids.long()))
    assert torch.equal(tsm.fused_moe_packed(x, p13, p2, w, ids), out)
    x, gw, w13, w2 = make_layer(9, 200, 16, 50, torch.bfloat16, seed=3)
    out = tsm.moe_forward(x, gw, w13, w2, 4, True)
    assert out.shape == (9, 200)
    w, ids, _ = tsm.moe_router(x, gw, 4, True)
    close(out, moe_reference(x, w13, w2, w, ids.long()))


def test_padded_pack_cache(tsm):
    """Reference-layout weights the kernels do not take as they are (I = 96) are packed with
    zero padding once per weight tensor: repeated calls reuse the copy, an in-place update of
    the weights rebuilds it, and the copy is dropped with the weights."""
    import gc
    from tinyserve_amd import ops
    x, gw, w13, w2 = make_layer(20, 256, 8, 96, torch.bfloat16, seed=4)
    w, ids, _ = tsm.moe_router(x, gw, 2, True)
    first = tsm.fused_moe(x, w13, w2, w, ids)
    entry = ops._padded_cache[id(w13)]
    again = tsm.fused_moe(x, w13, w2, w, ids)          # the repeated lookup
    assert torch.equal(first, again) and ops._padded_cache[id(w13)] is entry
    with torch.no_grad():
        w2.mul_(2)                                       # version moves: repacked
    twice = tsm.fused_moe(x, w13, w2, w, ids)
    assert ops._padded_cache[id(w13)] is not entry
    close(twice, moe_reference(x, w13, w2, w, ids.long()))
    assert not torch.equal(twice, first)
    key = id(w13)
    del w13, entry
    gc.collect()
    assert key not in ops._padded_cache


def test_fp32_layer(tsm):
    from oracle.moe_oracle import per_token_fp64
    x, gw, w13, w2 = make_layer(20, 256, 8, 512, torch.float32, seed=0)
    w, ids, _ = tsm.moe_router(x, gw, 2, True)
    out = tsm.fused_moe(x, w13, w2, w, ids)
    assert out.dtype == torch.float32
    r64 = per_token_fp64(x, w13, w2, w, ids.long())
    assert torch.allclose(out.double(), r64, atol=2e-6, rtol=1e-4)


@pytest.mark.parametrize("k,H", [(1, 256), (8, 256), (2, 4096), (1, 200)])
def test_add_rmsnorm(tsm, k, H):
    g = torch.Generator().manual_seed(k * H)
    rows = torch.randn(7 * k, H, generator=g).bfloat16()
    res = torch.randn(7, H, generator=g).bfloat16()
    nw = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    r = res.clone()
    out = tsm.ops.moe_combine_add_rmsnorm(rows, k, r, nw, 1e-6)
    ref, ref_res = add_rmsnorm_reference(rows, k, res, nw, 1e-6)
    assert torch.equal(r, ref_res)
    ulp = torch.exp2(torch.floor(torch.log2(ref.float().abs().clamp_min(2.0 ** -126))) - 7)
    assert bool(((out.float() - ref.float()).abs() <= ulp).all())
    if k == 1:   # without a residual: the norm of the rows themselves
        plain = tsm.ops.rmsnorm(rows, nw, 1e-6)
        pref = add_rmsnorm_reference(rows, 1, None, nw, 1e-6)[0]
        ulp = torch.exp2(torch.floor(torch.log2(pref.float().abs().clamp_min(2.0 ** -126))) - 7)
        assert bool(((plain.float() - pref.float()).abs() <= ulp).all())


def test_attention_side(tsm):
    from oracle.attn_oracle import paged_attention_ref, qk_norm_rope_ref
    from test_gpu_attn import Meta, build_batch
    from tinyserve_amd.attention import (PagedKVCache, greedy_argmax, paged_attention,
                                         qk_norm_rope)
    for H, Hkv, D, page, ql, kl in [(32, 4, 128, 16, [1, 1, 3, 0], [1, 33, 40, 0]),
                                    (8, 4, 64, 8, [3, 1, 17, 2], [9, 129, 17, 2]),
                                    (16, 1, 128, 32, [7, 1], [100, 300])]:
        q, kc, vc, cache, bt, qsl = build_batch("cpu", ql, kl, H, Hkv, D, page, seed=H + D)
        ref = paged_attention_ref(q.float(), kc.float(), vc.float(), qsl, kl, bt, D ** -0.5)
        for splits in (1, 4, 16):   # split-KV decode: 16 leaves splits empty at these lengths
            out = paged_attention(q, cache.k, cache.v, Meta("cpu", qsl, kl, bt), D ** -0.5,
                                  num_splits=splits).float()
            assert torch.isfinite(out).all()
            assert bool(((out - ref).abs() <= 8e-3 + ref.abs() * 2.0 ** -7).all()), splits
    T, H, Hkv, D = 5, 8, 2, 64
    g = torch.Generator().manual_seed(1)
    qkv = (torch.randn(T, (H + 2 * Hkv) * D, generator=g) * 3).bfloat16()
    ang = torch.rand(T, D // 2, generator=g) * 5
    qw = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    q, k, v = (t.reshape(T, -1, D) for t in qkv.split([H * D, Hkv * D, Hkv * D], -1))
    rq, rk = qk_norm_rope_ref(q, k, ang.cos(), ang.sin(), qw, kw, 1e-6)
    d = qkv.clone()
    dq, dk, dv = (t.view(T, -1, D) for t in d.split([H * D, Hkv * D, Hkv * D], -1))
    cache = PagedKVCache.allocate(4, 16, Hkv, D, "cpu")
    slots = torch.tensor([16, 17, 40, -1, 6000])          # -1 and past the pool: not written
    qk_norm_rope(dq, dk, ang.cos(), ang.sin(), qw, kw, 1e-6, dv, cache.k, cache.v, slots)
    assert torch.equal(dq, rq) and torch.equal(dk, rk)
    assert torch.equal(cache.k[1, 0], dk[0]) and torch.equal(cache.v[2, :, :, 8], v[2])
    x = torch.randn(6, 1000, generator=g)
    x[2, 5] = x[2, 900] = 99.0
    assert torch.equal(greedy_argmax(x), x.argmax(-1))


def test_end_to_end_driver(tsm):
    """The qwen3_moe driver (start-up plan tuning, prefill, then decode steps) on a two-layer
    model: its greedy tokens equal the decoder oracle's wherever the oracle's top two logits are
    apart."""
    from test_gpu_e2e import reference_logits, small_cfg
    from tinyserve_amd import kernels
    from tinyserve_amd.e2e import build_model, generate
    model = build_model(small_cfg(), device="cpu", seed=3, router_logits="fp32")
    prompts = torch.randint(0, 1000, (2, 20), generator=torch.Generator().manual_seed(7))
    try:
        plans = model.autotune(40, reps=1)     # the whole prefill: 2 x 20 tokens
        assert 1 << ((40 * model.cfg.num_experts_per_tok).bit_length() - 1) in plans
        toks, _, _ = generate(model, prompts, 4, graph=False)
    finally:
        kernels.set_moe_block_m(1, 1 << 30, -1, True)
        kernels.set_moe_block_m(1, 1 << 30, -1, False)
    ref, gaps = reference_logits(model, torch.cat([prompts, toks[:, :-1]], 1), True)
    steps = ref[:, 19:]
    top2 = steps.topk(2, dim=-1).values
    clear = ((top2[..., 0] - top2[..., 1]) > 3e-2 * steps.abs().max()) & (gaps[:, 19:] > 2e-3)
    assert bool((toks == steps.argmax(-1))[clear].all())


def test_packed_prefill_without_tile_kernels(tsm):
    """A layer the 128-row tile kernels do not take (2I % 256 != 0 here: H = 128, I = 64) at a
    prefill size: the plan must stay at 64-row tiles. (It once chose 128-row tiles whatever the
    shape, and the 64-row fallback kernel then read the 128-row permutation as 64-row tiles.)"""
    from tinyserve_amd import kernels
    T, H, E, I, k = 513, 128, 32, 64, 8
    assert kernels.moe_block_m(T, H, I, E, k, True) == 64
    x, gw, w13, w2 = make_layer(T, H, E, I, torch.bfloat16, seed=T)
    bias = torch.zeros(E)
    bias[E // 2:] = float("-inf")
    w, ids, _ = tsm.moe_router(x, gw, k, True, None, bias)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    out = tsm.fused_moe_packed(x, p13, p2, w, ids)
    assert torch.equal(out, tsm.fused_moe(x, w13, w2, w, ids))
    sel = slice(0, 64)
    close(out[sel], moe_reference(x[sel], w13, w2, w[sel], ids[sel].long()))
