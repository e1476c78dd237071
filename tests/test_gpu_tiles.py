"""The stage entry points (align, gate_up, down, combine) at the pipelined tile heights.

The 64-, 128- and 256-row tile kernels accumulate each output over K in one fp32 chain in the
same order, so their outputs are equal bit for bit; the result also equals the planned
fused_moe_packed at the same batch (a tile-kernel size) and, at a small batch, the oracle within
the bf16 tolerance."""
import pytest
import torch

from oracle.moe_oracle import make_layer, moe_reference

pytestmark = pytest.mark.gpu


def staged(tsm, x, p13, p2, w, ids, E, I, bm):
    from tinyserve_amd import _lib
    L = _lib.lib
    T, H = x.shape
    k = ids.shape[1]
    numel = T * k
    dev = x.device
    mp = int(L.tsm_moe_max_padded(numel, E, bm))
    nws = int(L.tsm_moe_align_workspace_size(numel, E, bm))
    sorted_ids = torch.empty(mp, dtype=torch.int32, device=dev)
    eids = torch.empty(mp // bm, dtype=torch.int32, device=dev)
    total = torch.empty(1, dtype=torch.int32, device=dev)
    aws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
    act = torch.empty(mp, I, dtype=torch.bfloat16, device=dev)
    rows = torch.empty(numel, H, dtype=torch.bfloat16, device=dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    s = _lib.stream_of(x)
    P = _lib.ptr
    _lib.check(L.tsm_moe_align(P(ids), numel, E, bm, P(sorted_ids), P(eids), P(total), P(aws),
                               nws, s), "align")
    _lib.check(L.tsm_moe_gemm_gate_up(P(x), P(p13), P(sorted_ids), P(eids), P(total), numel, k,
                                      H, I, E, bm, 1, P(act), s), f"gate_up bm={bm}")
    _lib.check(L.tsm_moe_gemm_down(P(act), P(p2), P(w), P(sorted_ids), P(eids), P(total), numel,
                                   H, I, E, bm, 1, P(rows), s), f"down bm={bm}")
    _lib.check(L.tsm_moe_combine(P(rows), T, H, k, P(out), s), "combine")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("H,I,E,k,T", [(2048, 768, 128, 8, 2048), (2048, 768, 128, 8, 1024),
                                       (1024, 2816, 16, 2, 1500), (768, 384, 32, 4, 700)])
def test_tile_heights_agree(dev, tsm, H, I, E, k, T):
    print(f"tile heights H={H} I={I} E={E} k={k} T={T}", flush=True)
    x, gw, w13, w2 = make_layer(T, H, E, I, torch.bfloat16, seed=T + E, device=dev)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    w, ids, _ = tsm.moe_router(x, gw, k, True)
    outs = {bm: staged(tsm, x, p13, p2, w, ids, E, I, bm) for bm in (64, 128, 256)}
    assert torch.equal(outs[64], outs[128]), "64 vs 128"
    assert torch.equal(outs[128], outs[256]), "128 vs 256"
    fused = tsm.fused_moe_packed(x, p13, p2, w, ids)
    assert torch.equal(fused, outs[128])


@pytest.mark.parametrize("bm", [64, 128, 256])
def test_tile_heights_against_oracle(dev, tsm, bm):
    H, I, E, k, T = 768, 384, 32, 4, 40
    x, gw, w13, w2 = make_layer(T, H, E, I, torch.bfloat16, seed=5, device=dev)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    w, ids, _ = tsm.moe_router(x, gw, k, True)
    out = staged(tsm, x, p13, p2, w, ids, E, I, bm).float().cpu()
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long()).float()
    max_abs = (out - ref).abs().max().item()
    mean_rel = ((out - ref).abs().mean() / ref.abs().mean()).item()
    print(f"bm={bm} vs oracle: max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}", flush=True)
    assert max_abs <= 2e-2 and mean_rel <= 5e-3


@pytest.mark.parametrize("kind", ["skew_remote"])
def test_tile_heights_skewed_with_remote_slots(dev, tsm, kind):
    """Skewed routing (a hot expert spanning several tiles of every height, cold experts with a
    few rows, so 256-row tiles run as half tiles) with a quarter of the experts owned by
    another GPU (their slots' ids are -1: zero rows, no GEMM): all heights give the same bits,
    the remote slots contribute nothing, and the result matches the oracle."""
    H, I, E, k, T = 768, 384, 32, 4, 700
    print(f"tile heights {kind} H={H} I={I} E={E} k={k} T={T}", flush=True)
    x, gw, w13, w2 = make_layer(T, H, E, I, torch.bfloat16, seed=17, device=dev)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    bias = torch.zeros(E)
    bias[3] = 6.0        # expert 3 in nearly every token's top-k
    bias[11] = 3.0
    emap = torch.arange(E, dtype=torch.int64)
    emap[24:] = -1       # experts 24..31 live on another GPU
    w, ids, _ = tsm.moe_router(x, gw, k, True, emap.to(dev), bias.to(dev))
    c = torch.bincount(ids.cpu().long().flatten() + 1, minlength=E + 1)
    assert c[0] > 0 and c[1 + 3] > 512 and (c[1:][c[1:] > 0] < 128).any()  # remote, hot, cold
    outs = {bm: staged(tsm, x, p13, p2, w, ids, E, I, bm) for bm in (64, 128, 256)}
    assert torch.equal(outs[64], outs[128]), "64 vs 128"
    assert torch.equal(outs[128], outs[256]), "128 vs 256"
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long()).float()
    out = outs[256].float().cpu()
    max_abs = (out - ref).abs().max().item()
    mean_rel = ((out - ref).abs().mean() / ref.abs().mean()).item()
    print(f"{kind} vs oracle: max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}", flush=True)
    assert max_abs <= 2e-2 and mean_rel <= 5e-3
