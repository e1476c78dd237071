"""GPU parity: routing (moe_route, fused moe_router) against the C oracle.

Routing from given logits is bit-exact at every size. The fused router's logits are bit-exact
with the oracle's fixed summation order where the kernel uses that order (fp32 inputs, and bf16
batches up to 256 tokens); bf16 batches above 256 tokens compute the gate GEMM on the matrix cores,
whose logits are checked against float64 dot products within the fp32 accumulation bound
|l - l64| <= 2^-17 * sum_h |x_h g_h| (+ one bf16 ulp when the logits are rounded to bf16), and
whose ids and weights are bit-exact with the oracle's selection on those logits."""
import numpy as np
import pytest
import torch

from oracle import c_oracle

pytestmark = pytest.mark.gpu


def bf16_bits(t):
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


ROUTE_CASES = [(1, 128, 8), (8, 128, 8), (64, 128, 8), (256, 128, 8), (2048, 128, 8),
               (64, 8, 2), (33, 60, 4), (5, 512, 8), (7, 64, 64), (3, 1, 1)]


@pytest.mark.parametrize("T,E,k", ROUTE_CASES)
@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("ldt", [torch.float32, torch.bfloat16])
def test_route_from_logits_bitexact(dev, tsm, T, E, k, renorm, ldt):
    print(f"route T={T} E={E} k={k} renorm={renorm} {ldt}", flush=True)
    g = torch.Generator().manual_seed(T * 1000 + E)
    logits = (torch.randn(T, E, generator=g) * 2).to(ldt)
    w, ids = tsm.moe_route(logits.to(dev), k, renorm, None)
    ow, oids = c_oracle.route(logits.float().numpy(), k, renorm)
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert same_bits(w.cpu().numpy(), ow)


def test_route_ties_and_masks(dev, tsm):
    """All-equal logits -> ids 0..k-1; -inf experts never chosen before finite ones; heavy bf16
    ties; expert_map with remote (-1) experts."""
    T, E, k = 16, 128, 8
    logits = torch.zeros(T, E)
    logits[1] = torch.arange(E) % 3            # ties among many experts
    logits[2, 64:] = float("-inf")             # half masked
    logits[3] = torch.full((E,), -1e30)
    logits[4, ::2] = 5.0                       # 64-way tie at the top
    logits[5] = torch.linspace(-100, 0, E)     # underflowing tail
    emap = torch.arange(E, dtype=torch.int64)
    emap[E // 2:] = -1
    for m in (None, emap):
        w, ids = tsm.moe_route(logits.to(dev), k, True, None if m is None else m.to(dev))
        ow, oids = c_oracle.route(logits.numpy(), k, True, None if m is None else m.numpy())
        assert np.array_equal(ids.cpu().numpy(), oids)
        assert same_bits(w.cpu().numpy(), ow)
    assert list(oids[0]) == list(range(k))
    assert list(c_oracle.route(logits.numpy(), k, True)[1][4]) == list(range(0, 2 * k, 2))


MFMA_MIN_T = 257   # bf16 batches from this size on run the gate GEMM on the matrix cores


def check_mfma_logits(logits, x, gw, logits_bf16=False, bias=None):
    """Kernel logits [T, E] against float64 dot products within the accumulation bound."""
    xd, gd = x.cpu().double(), gw.cpu().double()
    exact = xd @ gd.t()
    if bias is not None:
        exact = exact + bias.cpu().double()
    bound = (xd.abs() @ gd.abs().t()) * 2.0 ** -17 + 1e-30
    got = logits.cpu().double()
    if logits_bf16:
        ulp = torch.exp2(torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 7)
        bound = bound + ulp
        assert torch.equal(logits.cpu(), logits.cpu().bfloat16().float())
    assert bool(((got - exact).abs() <= bound).all()), float(((got - exact).abs() / bound).max())


@pytest.mark.parametrize("T", [1, 8, 64, 256, 300, 2048])
@pytest.mark.parametrize("logits_bf16", [False, True])
def test_router_fused_bitexact(dev, tsm, qwen_layer, T, logits_bf16):
    print(f"router T={T} logits_bf16={logits_bf16}", flush=True)
    (gate_w, _, _), (gate_c, _, _) = qwen_layer
    g = torch.Generator(device=dev).manual_seed(T)
    x = torch.randn(T, 2048, generator=g, device=dev).bfloat16()
    w, ids, logits = tsm.moe_router(x, gate_w, 8, True, None, None, logits_bf16)
    if T >= MFMA_MIN_T:
        check_mfma_logits(logits, x, gate_c, logits_bf16)
        ol = logits.cpu().numpy()
    else:
        ol = c_oracle.router_logits(bf16_bits(x), bf16_bits(gate_c), logits_bf16=logits_bf16)
        assert same_bits(logits.cpu().numpy(), ol)
    ow, oids = c_oracle.route(ol, 8, True)
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert same_bits(w.cpu().numpy(), ow)


@pytest.mark.parametrize("T", [257, 1000, 4096])
def test_router_mfma_without_logits_buffer(dev, tsm, qwen_layer, T):
    """The matrix-core router selects in the same launch, so it needs no logits buffer; the
    ids and weights equal those of the call with one, and a ragged last tile (T % 64) is routed."""
    from tinyserve_amd import _lib
    print(f"router mfma no-buffer T={T}", flush=True)
    (gate_w, _, _), _ = qwen_layer
    g = torch.Generator(device=dev).manual_seed(200 + T)
    x = torch.randn(T, 2048, generator=g, device=dev).bfloat16()
    w, ids, _ = tsm.moe_router(x, gate_w, 8, True)
    w1, ids1 = torch.empty_like(w), torch.empty_like(ids)
    rc = _lib.lib.tsm_moe_router(_lib.ptr(x), _lib.ptr(gate_w), 1, T, 2048, 128, 8, 1, None, None,
                                 0, None, _lib.ptr(w1), _lib.ptr(ids1), _lib.stream_of(x))
    _lib.check(rc, "tsm_moe_router")
    torch.cuda.synchronize()
    assert torch.equal(ids1, ids) and same_bits(w1.cpu().numpy(), w.cpu().numpy())
    # each token's routing depends on its own row only: a permuted batch routes the same
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(T)).to(dev)
    wp, idsp, _ = tsm.moe_router(x[perm], gate_w, 8, True)
    assert torch.equal(idsp, ids[perm])


@pytest.mark.parametrize("H,E,k,dtype", [(256, 8, 2, torch.float32), (256, 8, 2, torch.bfloat16),
                                         (1024, 60, 4, torch.bfloat16), (4096, 16, 4,
                                                                         torch.float32),
                                         (136, 5, 3, torch.float32)])
@pytest.mark.parametrize("T", [37, 300])
def test_router_fused_shapes(dev, tsm, H, E, k, dtype, T):
    g = torch.Generator().manual_seed(H + E)
    x = torch.randn(T, H, generator=g).to(dtype)
    gw = (torch.randn(E, H, generator=g) * 0.05).to(dtype)
    bias = torch.randn(E, generator=g)
    emap = torch.arange(E, dtype=torch.int64).flip(0)
    w, ids, logits = tsm.moe_router(x.to(dev), gw.to(dev), k, False, emap.to(dev), bias.to(dev))
    if dtype == torch.bfloat16 and T >= MFMA_MIN_T and H % 128 == 0:
        check_mfma_logits(logits, x, gw, bias=bias)
        ol = logits.cpu().numpy()
    elif dtype == torch.bfloat16:
        ol = c_oracle.router_logits(bf16_bits(x), bf16_bits(gw), bias=bias.numpy())
    else:
        ol = c_oracle.router_logits(x.numpy(), gw.numpy(), bias=bias.numpy())
    if not (dtype == torch.bfloat16 and T >= MFMA_MIN_T and H % 128 == 0):
        assert same_bits(logits.cpu().numpy(), ol)
    ow, oids = c_oracle.route(ol, k, False, emap.numpy())
    assert np.array_equal(ids.cpu().numpy(), oids)
    assert same_bits(w.cpu().numpy(), ow)


@pytest.mark.parametrize("T", [128, 1024])
def test_router_matches_torch_closed_form(dev, tsm, qwen_layer, T):
    """Independent of the oracle: logits vs float64 matmul, weights vs torch softmax/top-k."""
    (gate_w, _, _), (gate_c, _, _) = qwen_layer
    x = torch.randn(T, 2048, device=dev).bfloat16()
    w, ids, logits = tsm.moe_router(x, gate_w, 8, True)
    ref = x.cpu().double() @ gate_c.double().t()
    assert torch.allclose(logits.cpu().double(), ref, atol=1e-5, rtol=1e-5)
    p = logits.cpu().softmax(-1)
    tw = torch.gather(p, 1, ids.cpu().long())
    tw = tw / tw.sum(-1, keepdim=True)
    assert torch.allclose(w.cpu(), tw, atol=2e-6, rtol=1e-5)
    assert bool((w[:, :-1] >= w[:, 1:]).all())


@pytest.mark.parametrize("T", [1, 64, 256])
@pytest.mark.parametrize("logits_bf16", [False, True])
def test_router_single_launch_without_logits_buffer(dev, tsm, qwen_layer, T, logits_bf16):
    """tsm_moe_router without a logits buffer (one kernel per token) gives the same bits as with
    one (the gate GEMM split over expert slices, then selection from the buffer)."""
    from tinyserve_amd import _lib
    print(f"router single-launch T={T} logits_bf16={logits_bf16}", flush=True)
    (gate_w, _, _), _ = qwen_layer
    g = torch.Generator(device=dev).manual_seed(100 + T)
    x = torch.randn(T, 2048, generator=g, device=dev).bfloat16()
    w, ids, _ = tsm.moe_router(x, gate_w, 8, True, None, None, logits_bf16)
    w1 = torch.empty_like(w)
    ids1 = torch.empty_like(ids)
    rc = _lib.lib.tsm_moe_router(_lib.ptr(x), _lib.ptr(gate_w), 1, T, 2048, 128, 8, 1, None, None,
                                 int(logits_bf16), None, _lib.ptr(w1), _lib.ptr(ids1),
                                 _lib.stream_of(x))
    _lib.check(rc, "tsm_moe_router")
    torch.cuda.synchronize()
    assert torch.equal(ids1, ids)
    assert same_bits(w1.cpu().numpy(), w.cpu().numpy())
