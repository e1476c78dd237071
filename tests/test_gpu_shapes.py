"""Other MoE shapes through every path the plan picks (decode streaming tiles, expert-major,
64/128-row tiles, both weight layouts): outputs against the oracle at small batches, and the
packed and reference layouts against each other bit for bit at a tile-kernel batch."""
import pytest
import torch

from oracle.moe_oracle import make_layer, moe_reference

pytestmark = pytest.mark.gpu


def close(out, ref, what):
    out, ref = out.float().cpu(), ref.float().cpu()
    max_abs = (out - ref).abs().max().item()
    mean_rel = ((out - ref).abs().mean() / ref.abs().mean().clamp_min(1e-30)).item()
    print(f"{what}: max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}", flush=True)
    assert torch.isfinite(out).all() and max_abs <= 2e-2 and mean_rel <= 5e-3, what


# (H, I, E, top_k): a Qwen3-235B-like layer with half the experts, a wide-intermediate layer,
# and a small layer whose sizes miss the expert-major kernel table
@pytest.mark.parametrize("H,I,E,k", [(4096, 1536, 64, 8), (1024, 2816, 16, 2), (768, 384, 32, 4)])
def test_other_shapes(dev, tsm, H, I, E, k):
    print(f"shape H={H} I={I} E={E} k={k}", flush=True)
    x, gw, w13, w2 = make_layer(640, H, E, I, torch.bfloat16, seed=H + I, device=dev)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    w13c, w2c = w13.cpu(), w2.cpu()
    for T in (3, 40, 640):
        xs = x[:T].contiguous()
        w, ids, _ = tsm.moe_router(xs, gw, k, True)
        out = tsm.fused_moe(xs, w13, w2, w, ids)
        outp = tsm.fused_moe_packed(xs, p13, p2, w, ids)
        assert torch.equal(out, outp), (H, I, E, k, T)
        if T <= 40:
            close(out, moe_reference(xs.cpu(), w13c, w2c, w.cpu(), ids.cpu().long()),
                  f"H={H} I={I} E={E} k={k} T={T}")
