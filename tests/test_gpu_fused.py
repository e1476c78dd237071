"""GPU parity: the expert path (fused_moe, moe_forward, silu_and_mul) against the torch-CPU
oracle restatement of the reference's moe_reference (serve.py:933-996).

Tolerance (bf16 outputs): max |out - ref| <= 2e-2 and mean|out - ref| / mean|ref| <= 5e-3.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import c_oracle
from oracle.moe_oracle import moe_reference, moe_rows_reference

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_REL = 2e-2, 5e-3


def assert_close(out, ref, what=""):
    out, ref = out.float().cpu(), ref.float().cpu()
    assert torch.isfinite(out).all(), what
    max_abs = (out - ref).abs().max().item()
    mean_rel = ((out - ref).abs().mean() / ref.abs().mean().clamp_min(1e-30)).item()
    print(f"{what}: max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}", flush=True)
    assert max_abs <= MAX_ABS, (what, max_abs)
    assert mean_rel <= MEAN_REL, (what, mean_rel)


def xrand(T, H, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(T, H, generator=g, device=dev).bfloat16()


@pytest.mark.parametrize("T", [1, 8, 64, 256, 512, 2048])
def test_fused_moe_qwen_shape(dev, tsm, qwen_layer, T):
    print(f"fused_moe qwen T={T}", flush=True)
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    x = xrand(T, 2048, dev, T)
    w, ids, _ = tsm.moe_router(x, gw, 8, True)
    out = tsm.fused_moe(x, w13, w2, w, ids)
    ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
    assert_close(out, ref, f"T={T}")


@pytest.mark.emu_tokens(8192)
def test_fused_moe_full_size_token_subset(dev, tsm, qwen_layer):
    """T=8192 (largest prefill config): every token's output depends only on its own row, so the
    oracle on a sampled subset of tokens checks the full-size launch exactly."""
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    T = 8192
    x = xrand(T, 2048, dev, 99)
    w, ids, _ = tsm.moe_router(x, gw, 8, True)
    out = tsm.fused_moe(x, w13, w2, w, ids)
    sel = torch.randperm(T, generator=torch.Generator().manual_seed(0))[:384]
    ref = moe_reference(x.cpu()[sel], w13c, w2c, w.cpu()[sel], ids.cpu().long()[sel])
    assert_close(out.cpu()[sel], ref, "T=8192 subset")
    # the packed-weight prefill kernels (persistent 128-row tiles) give the same bits in full
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    assert torch.equal(tsm.fused_moe_packed(x, p13, p2, w, ids), out)


def test_rows_sum_topk_false(dev, tsm, qwen_layer):
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    x = xrand(64, 2048, dev, 5)
    w, ids, _ = tsm.moe_router(x, gw, 8, True)
    rows = tsm.fused_moe(x, w13, w2, w, ids, sum_topk=False)
    assert rows.shape == (64 * 8, 2048)
    ref = moe_rows_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
    assert_close(rows, ref, "rows")
    # the k-sum of the rows is the summed output, bit for bit
    summed = tsm.fused_moe(x, w13, w2, w, ids)
    assert torch.equal(summed.cpu(), rows.cpu().float().view(64, 8, 2048).sum(1).bfloat16())


@pytest.mark.parametrize("T", [3, 64, 700])
def test_expert_parallel_remote_ids(dev, tsm, qwen_layer, T):
    """expert_map sends half the experts to 'another GPU' (-1): their rows are zero."""
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    x = xrand(T, 2048, dev, 7 + T)
    emap = torch.arange(128, dtype=torch.int64, device=dev)
    emap[64:] = -1
    w, ids, _ = tsm.moe_router(x, gw, 8, True, emap)
    assert bool((ids.cpu() < 64).all()) and bool((ids.cpu() >= -1).all())
    out = tsm.fused_moe(x, w13, w2, w, ids)
    ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
    assert_close(out, ref, f"EP T={T}")
    rows = tsm.fused_moe(x, w13, w2, w, ids, sum_topk=False).cpu().view(T, 8, 2048)
    assert bool((rows[ids.cpu() < 0] == 0).all())


@pytest.mark.emu_tokens(2048)
@pytest.mark.parametrize("kind", ["zipf", "half_empty"])
def test_load_imbalance(dev, tsm, qwen_layer, kind):
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    T = 2048
    x = xrand(T, 2048, dev, 11)
    gen = torch.Generator().manual_seed(1)
    if kind == "zipf":
        p = 1.0 / torch.arange(1, 129, dtype=torch.float64) ** 1.2
        p = p[torch.randperm(128, generator=gen)]
        bias = torch.log(p / p.sum()).float()
    else:
        bias = torch.zeros(128)
        bias[64:] = float("-inf")
    w, ids, _ = tsm.moe_router(x, gw, 8, True, None, bias.to(dev))
    counts = torch.bincount(ids.cpu().long().flatten(), minlength=128)
    if kind == "zipf":
        assert counts.max().item() > 10 * counts.float().mean().item()
    else:
        assert counts[64:].sum().item() == 0
    out = tsm.fused_moe(x, w13, w2, w, ids)
    ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
    assert_close(out, ref, kind)
    # the default product path (packed weights: persistent 128-row tiles at this size, hot
    # experts spanning many tiles) gives the same bits, and so matches the oracle too
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    packed = tsm.fused_moe_packed(x, p13, p2, w, ids)
    assert torch.equal(packed, out), kind
    assert_close(packed, ref, f"{kind} packed")
    whole = tsm.moe_forward_packed(x, gw, p13, p2, 8, True, None, bias.to(dev))
    assert torch.equal(whole, out), kind


@pytest.mark.parametrize("T", [1, 37, 64])
def test_tiny_config_bf16(dev, tsm, T):
    """Config-0 shape (H=256, E=8, top-2, I=512) in bf16."""
    from oracle.moe_oracle import make_layer
    x, gw, w13, w2 = make_layer(T, 256, 8, 512, torch.bfloat16, seed=0, device=dev)
    w, ids, _ = tsm.moe_router(x, gw, 2, True)
    out = tsm.fused_moe(x, w13, w2, w, ids)
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long())
    assert_close(out, ref, f"tiny T={T}")


def test_moe_forward_matches_composition_and_is_deterministic(dev, tsm, qwen_layer):
    (gw, w13, w2), _ = qwen_layer
    x = xrand(200, 2048, dev, 3)
    a = tsm.moe_forward(x, gw, w13, w2, 8, True)
    b = tsm.moe_forward(x, gw, w13, w2, 8, True)
    w, ids, _ = tsm.moe_router(x, gw, 8, True)
    c = tsm.fused_moe(x, w13, w2, w, ids)
    assert torch.equal(a, b) and torch.equal(a, c)


def test_reference_style_router_path(dev, tsm, qwen_layer):
    """SparseMoE(router='linear'): bf16 nn.Linear logits -> moe_route -> fused_moe, as the
    reference's forward composes them (serve.py:1079-1087)."""
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    x = xrand(64, 2048, dev, 4)
    logits = F.linear(x, gw)
    w, ids = tsm.moe_route(logits, 8, True, torch.arange(128, device=dev))
    ow, oids = c_oracle.route(logits.float().cpu().numpy(), 8, True)
    assert np.array_equal(ids.cpu().numpy(), oids)
    out = tsm.fused_moe(x, w13, w2, w, ids)
    ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
    assert_close(out, ref, "linear router")


def test_sparse_moe_module(dev, tsm, qwen_layer):
    """The module mirror of serve.py SparseMoE, with both router modes; the oracle is given the
    routing the module used (routing parity itself is pinned bit-exactly by test_gpu_route)."""
    from types import SimpleNamespace
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    cfg = SimpleNamespace(num_experts=128, hidden_size=2048, moe_intermediate_size=768,
                          num_experts_per_tok=8, norm_topk_prob=True)
    x = xrand(16, 2048, dev, 8)
    for router, packed in (("fused", True), ("linear", True), ("fused", False),
                           ("linear", False)):
        m = tsm.SparseMoE(cfg, router=router, packed=packed).to(device=dev,
                                                                dtype=torch.bfloat16)
        with torch.no_grad():
            m.gate.weight.copy_(gw)
            m.w13.copy_(w13)
            m.w2.copy_(w2)
            out = m(x)
            if router == "fused":
                # a bf16 module rounds its logits to bf16, as the reference's bf16 Linear does
                w, ids, _ = tsm.moe_router(x, gw, 8, True, None, None, True)
            else:
                w, ids = tsm.moe_route(m.gate(x), 8, True, m.expert_map)
        ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
        assert_close(out, ref, f"SparseMoE {router} packed={packed}")
        # the module holds one copy of its expert weights and hands back the reference layout
        if packed:
            assert m.weights_packed
            sd = m.state_dict()
            assert torch.equal(sd["w13"], w13) and torch.equal(sd["w2"], w2)


def test_moe_forward_bf16_logits_mode(dev, tsm, qwen_layer):
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    x = xrand(64, 2048, dev, 9)
    out = tsm.moe_forward(x, gw, w13, w2, 8, True, None, None, True)
    w, ids, logits = tsm.moe_router(x, gw, 8, True, None, None, True)
    assert torch.equal(logits, logits.bfloat16().float())
    ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
    assert_close(out, ref, "bf16 logits")


@pytest.mark.emu_skip("HIP graph capture")
def test_graph_capture_replay(dev, tsm, qwen_layer):
    """The op captures into a HIP graph (static grid, no host sync, no allocation in the C ABI);
    each replay, with eager work in between, matches the eager result bit for bit."""
    (gw, w13, w2), _ = qwen_layer
    x = xrand(64, 2048, dev, 21)
    eager = tsm.moe_forward(x, gw, w13, w2, 8, True)
    static_x = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        tsm.moe_forward(static_x, gw, w13, w2, 8, True)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = tsm.moe_forward(static_x, gw, w13, w2, 8, True)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), i
        junk = tsm.moe_forward(xrand(17, 2048, dev, 100 + i), gw, w13, w2, 8, True)
        torch.cuda.synchronize()
        del junk
    static_x.copy_(xrand(64, 2048, dev, 22))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(static_out, tsm.moe_forward(static_x, gw, w13, w2, 8, True))


def test_silu_and_mul(dev, tsm):
    """Against the oracle restatement (tinykernels.py:293-297): equal except where the kernel's
    hardware sigmoid lands the rounded silu on the other side of a bf16 rounding boundary
    (then within one bf16 ulp of the product)."""
    from oracle.moe_oracle import silu_and_mul_reference
    g = torch.randn(300, 2 * 768, device=dev).bfloat16() * 3
    out = tsm.silu_and_mul(g[:, :768], g[:, 768:])
    ref = silu_and_mul_reference(g[:, :768].cpu(), g[:, 768:].cpu())
    diff = (out.float().cpu() - ref.float()).abs()
    ulp = ref.float().abs().clamp_min(1e-30) * 2.0 ** -6  # two bf16 ulps
    assert bool((diff <= ulp + 1e-30).all())
    assert (diff > 0).float().mean().item() < 1e-2


def test_pack_layout_matches_definition(dev, tsm):
    """packed[e][blk][s][lane][i] = W[e][16*src(blk) + lane%16][32*s + 8*(lane//16) + i]."""
    E, I, H = 3, 64, 256
    w13 = torch.randn(E, 2 * I, H, device=dev).bfloat16()
    w2 = torch.randn(E, H, I, device=dev).bfloat16()
    p13, p2 = tsm.pack_moe_weights(w13, w2)

    def ref(W, interleave):
        E_, N, K = W.shape
        blocks = W.view(E_, N // 16, 16, K // 32, 4, 8)            # e, blk, r, s, q, i
        if interleave:
            nb = N // 16
            order = [j // 2 if j % 2 == 0 else nb // 2 + j // 2 for j in range(nb)]
            blocks = blocks[:, order]
        return blocks.permute(0, 1, 3, 4, 2, 5).reshape(E_, N, K)  # e, blk, s, lane=(q,r), i

    assert torch.equal(p13.cpu(), ref(w13.cpu(), True))
    assert torch.equal(p2.cpu(), ref(w2.cpu(), False))


@pytest.mark.parametrize("T", [1, 8, 64, 256, 512, 2048, 4096])
def test_packed_path_bitexact_with_reference_layout(dev, tsm, qwen_layer, T):
    """The packed kernels consume the same k order per lane as the reference-layout kernels, so
    outputs are identical bit for bit; and both match the oracle."""
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    x = xrand(T, 2048, dev, 40 + T)
    a = tsm.moe_forward(x, gw, w13, w2, 8, True)
    b = tsm.moe_forward_packed(x, gw, p13, p2, 8, True)
    assert torch.equal(a, b)
    w, ids, _ = tsm.moe_router(x, gw, 8, True)
    rows = tsm.fused_moe_packed(x, p13, p2, w, ids, sum_topk=False)
    assert torch.equal(rows, tsm.fused_moe(x, w13, w2, w, ids, sum_topk=False))
    if T <= 256:
        ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
        assert_close(b, ref, f"packed T={T}")


@pytest.mark.emu_tokens(3200)
def test_packed_expert_parallel_and_tiny(dev, tsm, qwen_layer):
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    emap = torch.arange(128, dtype=torch.int64, device=dev)
    emap[::2] = -1
    for T in (50, 700, 3200):  # weight-streaming, 128-row and 256-row tile kernels
        x = xrand(T, 2048, dev, 77)
        w, ids, _ = tsm.moe_router(x, gw, 8, True, emap)
        out = tsm.fused_moe_packed(x, p13, p2, w, ids)
        assert torch.equal(out, tsm.fused_moe(x, w13, w2, w, ids)), f"packed EP T={T}"
        if T <= 700:  # the CPU reference is slow beyond this; above it the bit-exact match with
            ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())  # the layout
            assert_close(out, ref, f"packed EP T={T}")  # checked at T=700 carries parity
    from oracle.moe_oracle import make_layer
    x, gw, w13, w2 = make_layer(37, 256, 8, 512, torch.bfloat16, seed=0, device=dev)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    w, ids, _ = tsm.moe_router(x, gw, 2, True)
    out = tsm.fused_moe_packed(x, p13, p2, w, ids)
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long())
    assert_close(out, ref, "packed tiny")
    # tiny shape at a tile-kernel batch (K = 256 and 512: short pipelines)
    x = xrand(2048, 256, dev, 78)
    w, ids, _ = tsm.moe_router(x, gw, 2, True)
    out = tsm.fused_moe_packed(x, p13, p2, w, ids)
    assert torch.equal(out, tsm.fused_moe(x, w13, w2, w, ids))
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long())
    assert_close(out, ref, "packed tiny T=2048")


@pytest.mark.parametrize("T", [512, 2048])
def test_packed_prefill_against_oracle(dev, tsm, qwen_layer, T):
    """Prefill sizes on the default (packed) path against the oracle directly: T=512 runs the
    64-row tile kernels, T=2048 the 128-row persistent tiles (a token subset is checked there;
    each token's output depends only on its own row)."""
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    x = xrand(T, 2048, dev, 300 + T)
    w, ids, _ = tsm.moe_router(x, gw, 8, True)
    out = tsm.moe_forward_packed(x, gw, p13, p2, 8, True)
    sel = torch.arange(T) if T <= 512 else \
        torch.randperm(T, generator=torch.Generator().manual_seed(T))[:512]
    ref = moe_reference(x.cpu()[sel], w13c, w2c, w.cpu()[sel], ids.cpu().long()[sel])
    assert_close(out.cpu()[sel], ref, f"packed prefill T={T}")


def test_pack_padded_matches_layout_definition(dev, tsm):
    """The HIP packing kernel, with and without zero padding, against the tensor-permutation
    statement of the layout (tinyserve_amd.layout, pinned on the CPU by test_layout), and the
    inverse permutation restores the weights."""
    from tinyserve_amd import layout
    for E, I, H in ((3, 64, 256), (2, 96, 256), (2, 24, 200), (1, 50, 136)):
        g = torch.Generator(device=dev).manual_seed(E * I + H)
        w13 = torch.randn(E, 2 * I, H, generator=g, device=dev).bfloat16()
        w2 = torch.randn(E, H, I, generator=g, device=dev).bfloat16()
        Hp, Ip = tsm.ops.padded_shape(H, I)
        p13, p2 = tsm.pack_moe_weights(w13, w2)
        assert tuple(p13.shape) == (E, 2 * Ip, Hp) and tuple(p2.shape) == (E, Hp, Ip)
        assert torch.equal(p13.cpu(), layout.pack(w13.cpu(), True, 2 * Ip, Hp)), (E, I, H)
        assert torch.equal(p2.cpu(), layout.pack(w2.cpu(), False, Hp, Ip)), (E, I, H)
        assert torch.equal(layout.unpack(p13, True, 2 * I, H), w13)
        assert torch.equal(layout.unpack(p2, False, H, I), w2)


@pytest.mark.parametrize("T", [1, 64, 700, 2048])
def test_tp8_share_intermediate_96(dev, tsm, T):
    """The one-GPU share of TP-8 for Qwen3-30B-A3B: I = 768 / 8 = 96, which the kernels run
    zero-padded to 128 (the reference masks the ragged block instead, tinykernels.py:1719-1731).
    Both the reference-layout op and the packed path against the oracle."""
    from oracle.moe_oracle import make_layer
    _, gw, w13, w2 = make_layer(1, 2048, 128, 96, torch.bfloat16, seed=5, device=dev)
    x = xrand(T, 2048, dev, 500 + T)
    w, ids, _ = tsm.moe_router(x, gw, 8, True)
    out = tsm.fused_moe(x, w13, w2, w, ids)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    assert tuple(p2.shape) == (128, 2048, 128)
    assert torch.equal(tsm.fused_moe_packed(x, p13, p2, w, ids), out)
    assert torch.equal(tsm.moe_forward_packed(x, gw, p13, p2, 8, True), out)
    rows = tsm.fused_moe(x, w13, w2, w, ids, sum_topk=False)
    assert rows.shape == (T * 8, 2048)
    sel = torch.arange(T) if T <= 700 else \
        torch.randperm(T, generator=torch.Generator().manual_seed(T))[:512]
    ref = moe_reference(x.cpu()[sel], w13.cpu(), w2.cpu(), w.cpu()[sel], ids.cpu().long()[sel])
    assert_close(out.cpu()[sel], ref, f"I=96 T={T}")


@pytest.mark.parametrize("T", [5, 300])
def test_ragged_hidden_size(dev, tsm, T):
    """H = 200 (not a multiple of 128) and I = 50: x is zero-padded to H_pad = 256 for the
    experts and the output cut back to H; the router runs on the true H (padded to a multiple
    of 8 with zero columns, which leaves its sums unchanged)."""
    from oracle.moe_oracle import make_layer
    E, k = 16, 4
    x, gw, w13, w2 = make_layer(T, 200, E, 50, torch.bfloat16, seed=6, device=dev)
    w, ids, logits = tsm.moe_router(x, gw, k, True)
    bits = lambda t: t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    ol = c_oracle.router_logits(bits(x), bits(gw))
    assert np.array_equal(logits.cpu().numpy().view(np.uint32), ol.view(np.uint32))
    out = tsm.moe_forward(x, gw, w13, w2, k, True)
    assert out.shape == (T, 200)
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long())
    assert_close(out, ref, f"H=200 T={T}")
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    assert torch.equal(tsm.moe_forward_packed(x, gw, p13, p2, k, True), out)


def test_module_routes_like_bf16_linear(dev, tsm, qwen_layer):
    """SparseMoE (bf16) routes on bf16-rounded logits, as serve.py's bf16 nn.Linear gate does
    (serve.py:1079): its ids equal the oracle's selection on the bf16 logits of the module's own
    router, and those logits agree with torch's bf16 Linear to within one bf16 ulp (the GEMM
    libraries sum in another order, so a logit near a rounding boundary may round the other way).
    The input is tie-prone: repeated token rows and a gate with duplicated expert rows."""
    from types import SimpleNamespace
    (gw, w13, w2), _ = qwen_layer
    gw_t = gw.clone()
    gw_t[1::2] = gw_t[0::2]                      # experts 2j and 2j+1 always tie
    x = xrand(32, 2048, dev, 61).repeat(2, 1)
    w, ids, logits = tsm.moe_router(x, gw_t, 8, True, None, None, True)
    ow, oids = c_oracle.route(logits.cpu().numpy(), 8, True)
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), ow.view(np.uint32))
    # ties resolve to the lower expert index
    assert bool((ids.cpu()[:, 0] % 2 == 0).all())
    lin = F.linear(x, gw_t).float()
    d = (lin - logits).abs()
    ulp = logits.abs().clamp_min(2.0 ** -126) * 2.0 ** -7
    assert bool((d <= ulp).all())
    assert (d > 0).float().mean().item() < 1e-2
    cfg = SimpleNamespace(num_experts=128, hidden_size=2048, moe_intermediate_size=768,
                          num_experts_per_tok=8, norm_topk_prob=True)
    m = tsm.SparseMoE(cfg).to(device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        m.gate.weight.copy_(gw_t)
        m.w13.copy_(w13)
        m.w2.copy_(w2)
        out = m(x)
    assert torch.equal(out, tsm.fused_moe(x, w13, w2, w, ids))


@pytest.mark.parametrize("T", [64, 1, 300])
def test_tiny_config_fp32(dev, tsm, T):
    """Config 1 as specified: H=256, E=8, top-2, I=512, fp32 throughout (x ~ N(0,1), weights
    ~ N(0, 0.02), seed 0): the fp32 router and the fp32 experts against the fp32 oracle (same
    routing) and the float64 per-token formula."""
    from types import SimpleNamespace
    from oracle.moe_oracle import make_layer, per_token_fp64, route_torch
    x, gw, w13, w2 = make_layer(T, 256, 8, 512, torch.float32, seed=0, device=dev)
    w, ids, logits = tsm.moe_router(x, gw, 2, True)
    rw, rids = route_torch(logits.cpu(), 2, True)
    assert torch.equal(ids.cpu().long(), rids)
    out = tsm.fused_moe(x, w13, w2, w, ids)
    assert out.dtype == torch.float32
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long())
    assert torch.allclose(out.cpu(), ref, atol=2e-6, rtol=1e-4), (out.cpu() - ref).abs().max()
    r64 = per_token_fp64(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long())
    assert torch.allclose(out.cpu().double(), r64, atol=2e-6, rtol=1e-4)
    rows = tsm.fused_moe(x, w13, w2, w, ids, sum_topk=False)
    assert torch.equal(rows.view(T, 2, 256)[:, 0] + rows.view(T, 2, 256)[:, 1], out)
    assert torch.equal(tsm.moe_forward(x, gw, w13, w2, 2, True), out)
    cfg = SimpleNamespace(num_experts=8, hidden_size=256, moe_intermediate_size=512,
                          num_experts_per_tok=2, norm_topk_prob=True)
    m = tsm.SparseMoE(cfg).to(dev)
    with torch.no_grad():
        m.gate.weight.copy_(gw)
        m.w13.copy_(w13)
        m.w2.copy_(w2)
        assert torch.equal(m(x), out)


@pytest.mark.emu_skip("times every plan on the full layer up to 512 tokens (the emulated "
                      "kernel suite tunes a small layer instead)")
def test_autotune_installs_plans(dev, tsm, qwen_layer):
    """autotune_fused_moe times the candidate tile heights per batch-size bucket and installs
    the fastest; the plans it installs keep parity with the oracle, and clearing them restores
    the static table."""
    from tinyserve_amd import kernels
    (gw, w13, w2), (_, w13c, w2c) = qwen_layer
    before = {T: kernels.moe_block_m(T, 2048, 768, 128, 8) for T in (1, 64, 512)}
    table = kernels.autotune_fused_moe(w13, w2, 8, 512)
    assert set(table) == {1 << (n.bit_length() - 1) for n in (8, 16, 32, 64, 128, 256, 512,
                                                                 1024, 2048, 4096)}
    for T in (1, 64, 512):
        bm, _ = table[1 << ((T * 8).bit_length() - 1)]
        assert kernels.moe_block_m(T, 2048, 768, 128, 8) == bm
        x = xrand(T, 2048, dev, 900 + T)
        w, ids, _ = tsm.moe_router(x, gw, 8, True)
        ref = moe_reference(x.cpu(), w13c, w2c, w.cpu(), ids.cpu().long())
        assert_close(tsm.fused_moe(x, w13, w2, w, ids), ref, f"autotuned T={T} bm={bm}")
    kernels.set_moe_block_m(1, 1 << 30, -1)
    assert {T: kernels.moe_block_m(T, 2048, 768, 128, 8) for T in (1, 64, 512)} == before


def test_packed_prefill_without_tile_kernels(dev, tsm):
    """A layer the 128-row tile kernels do not take (H = 128, I = 64: 2I % 256 != 0) at a
    prefill size runs 64-row tiles on packed weights and matches the reference layout and the
    oracle (the plan once chose 128-row tiles whatever the shape)."""
    from oracle.moe_oracle import make_layer
    T, H, E, I, k = 1500, 128, 32, 64, 8
    x, gw, w13, w2 = make_layer(T, H, E, I, torch.bfloat16, seed=T, device=dev)
    w, ids, _ = tsm.moe_router(x, gw, k, True)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    out = tsm.fused_moe_packed(x, p13, p2, w, ids)
    assert torch.equal(out, tsm.fused_moe(x, w13, w2, w, ids))
    sel = torch.arange(0, T, 5)
    ref = moe_reference(x.cpu()[sel], w13.cpu(), w2.cpu(), w.cpu()[sel], ids.cpu().long()[sel])
    assert_close(out.cpu()[sel], ref, "H=128 I=64 packed prefill")
