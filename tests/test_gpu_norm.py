"""GPU parity: residual-add RMSNorm and its fusion with the MoE top-k combine (moe_norm.hip)
against the oracle restatement of serve.py's RMSNorm / add_rmsnorm (add_rmsnorm_reference).

The residual stream is bit-exact (its arithmetic is the same bf16 roundings of fixed-order fp32
sums); the normalised output is within one bf16 ulp of the oracle (the kernel's reciprocal square
root and sum-of-squares order differ from torch's)."""
import pytest
import torch

from oracle.moe_oracle import add_rmsnorm_reference

pytestmark = pytest.mark.gpu


def ulp_close(out, ref):
    out, ref = out.double().cpu(), ref.double().cpu()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -126))) - 7)
    bad = (out - ref).abs() > ulp
    assert not bool(bad.any()), f"{int(bad.sum())} elements beyond 1 bf16 ulp"


@pytest.mark.parametrize("T,H", [(1, 2048), (64, 2048), (300, 4096), (5, 200), (3, 16384),
                                 (2, 8), (4096, 2048)])
def test_rmsnorm_with_and_without_residual(dev, tsm, T, H):
    print(f"rmsnorm T={T} H={H}", flush=True)
    g = torch.Generator(device=dev).manual_seed(T + H)
    x = torch.randn(T, H, generator=g, device=dev).bfloat16()
    res = (torch.randn(T, H, generator=g, device=dev) * 3).bfloat16()
    w = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).bfloat16()
    out = tsm.ops.rmsnorm(x, w, 1e-6)
    ref, _ = add_rmsnorm_reference(x.cpu(), 1, None, w.cpu(), 1e-6)
    ulp_close(out, ref)
    r = res.clone()
    out = tsm.ops.rmsnorm(x, w, 1e-6, r)
    ref, ref_res = add_rmsnorm_reference(x.cpu(), 1, res.cpu(), w.cpu(), 1e-6)
    assert torch.equal(r.cpu(), ref_res)
    ulp_close(out, ref)


@pytest.mark.parametrize("T", [1, 64, 2048, 8192])
def test_moe_combine_add_rmsnorm(dev, tsm, qwen_layer, T):
    """rows of the MoE block (sum_topk=False) -> combine + residual add + RMSNorm in one launch:
    the residual equals bf16(fused_moe output + residual) bit for bit."""
    print(f"combine+norm T={T}", flush=True)
    (gw, w13, w2), _ = qwen_layer
    g = torch.Generator(device=dev).manual_seed(T)
    x = torch.randn(T, 2048, generator=g, device=dev).bfloat16()
    res = torch.randn(T, 2048, generator=g, device=dev).bfloat16()
    nw = (1 + 0.1 * torch.randn(2048, generator=g, device=dev)).bfloat16()
    w, ids, _ = tsm.moe_router(x, gw, 8, True)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    rows = tsm.fused_moe_packed(x, p13, p2, w, ids, sum_topk=False)
    summed = tsm.fused_moe_packed(x, p13, p2, w, ids)
    r = res.clone()
    out = tsm.ops.moe_combine_add_rmsnorm(rows, 8, r, nw, 1e-6)
    assert torch.equal(r, (summed.float() + res.float()).bfloat16())
    sel = slice(0, min(T, 512))
    ref, ref_res = add_rmsnorm_reference(rows.cpu()[:min(T, 512) * 8], 8, res.cpu()[sel],
                                         nw.cpu(), 1e-6)
    assert torch.equal(r.cpu()[sel], ref_res)
    ulp_close(out.cpu()[sel], ref)
    # first layer form: no residual to add, the residual becomes the combined output
    r0 = torch.empty_like(res)
    out0 = tsm.ops.moe_combine_add_rmsnorm(rows, 8, r0, nw, 1e-6, residual_in=False)
    assert torch.equal(r0, summed)
    assert torch.equal(out0, tsm.ops.rmsnorm(summed, nw, 1e-6))
