"""Edge cases of the public ops: empty batches, every assignment owned by another GPU, a single
expert with top-1 routing, and the largest top_k (k = E)."""
import pytest
import torch

from oracle.moe_oracle import make_layer, moe_reference

pytestmark = pytest.mark.gpu


def test_empty_batch(dev, tsm, qwen_layer):
    (gw, w13, w2), _ = qwen_layer
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    x = torch.empty(0, 2048, dtype=torch.bfloat16, device=dev)
    w, ids, logits = tsm.moe_router(x, gw, 8, True)
    assert w.shape == (0, 8) and ids.shape == (0, 8) and logits.shape == (0, 128)
    assert tsm.fused_moe_packed(x, p13, p2, w, ids).shape == (0, 2048)
    assert tsm.fused_moe(x, w13, w2, w, ids, sum_topk=False).shape == (0, 2048)
    assert tsm.moe_forward_packed(x, gw, p13, p2, 8, True).shape == (0, 2048)
    sorted_ids, expert_ids, total = tsm.moe_align_block_size(ids, 16, 128)
    torch.cuda.synchronize()
    assert int(total.item()) == 0 and bool((expert_ids == -1).all())
    assert bool((sorted_ids == 0).all())  # every row is padding (value numel = 0)


@pytest.mark.parametrize("T", [8, 2048])
def test_all_assignments_remote(dev, tsm, qwen_layer, T):
    """expert_map sends every expert to another GPU: all rows and the output are zero."""
    print(f"all remote T={T}", flush=True)
    (gw, w13, w2), _ = qwen_layer
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    g = torch.Generator(device=dev).manual_seed(T)
    x = torch.randn(T, 2048, generator=g, device=dev).bfloat16()
    emap = torch.full((128,), -1, dtype=torch.int64, device=dev)
    w, ids, _ = tsm.moe_router(x, gw, 8, True, emap)
    assert bool((ids == -1).all())
    for packed in (False, True):
        a, b = (p13, p2) if packed else (w13, w2)
        fn = tsm.fused_moe_packed if packed else tsm.fused_moe
        rows = fn(x, a, b, w, ids, sum_topk=False)
        out = fn(x, a, b, w, ids)
        torch.cuda.synchronize()
        assert bool((rows == 0).all()) and bool((out == 0).all())


@pytest.mark.parametrize("T", [1, 40, 3000])
def test_single_expert_top1(dev, tsm, T):
    """E = 1, k = 1: every token goes to the one expert with weight 1."""
    print(f"single expert T={T}", flush=True)
    x, gw, w13, w2 = make_layer(T, 256, 1, 128, torch.bfloat16, seed=T, device=dev)
    w, ids, _ = tsm.moe_router(x, gw, 1, True)
    assert bool((ids == 0).all()) and bool((w == 1.0).all())
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long()).float()
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    for out in (tsm.fused_moe(x, w13, w2, w, ids), tsm.fused_moe_packed(x, p13, p2, w, ids)):
        out = out.float().cpu()
        assert (out - ref).abs().max().item() <= 2e-2
        assert ((out - ref).abs().mean() / ref.abs().mean()).item() <= 5e-3


def test_top_k_equals_experts(dev, tsm):
    """k = E = 8: every expert is selected, in descending-probability order."""
    T, H, E, I = 64, 256, 8, 512
    x, gw, w13, w2 = make_layer(T, H, E, I, torch.bfloat16, seed=3, device=dev)
    w, ids, logits = tsm.moe_router(x, gw, E, True)
    assert bool((ids.sort(dim=1).values == torch.arange(E, device=dev)).all())
    assert torch.allclose(w.sum(1), torch.ones(T, device=dev), atol=1e-6)
    assert bool((w[:, :-1] >= w[:, 1:]).all())
    ref = moe_reference(x.cpu(), w13.cpu(), w2.cpu(), w.cpu(), ids.cpu().long()).float()
    out = tsm.fused_moe(x, w13, w2, w, ids).float().cpu()
    assert (out - ref).abs().max().item() <= 2e-2
