"""A batch past the 32-bit element-offset range: T*H >= 2^32 (gate_up's gathered rows of x) and
padded rows * I >= 2^32 (down's rows of the activation buffer). Each output row depends only on
its own token row, its routing and the expert weights, so x repeating with period P must give
an output repeating with period P, every period equal bit for bit to the output of the first P
tokens alone."""
import pytest
import torch

from oracle.moe_oracle import make_layer

pytestmark = pytest.mark.gpu

H, I, E, K, P = 2048, 768, 16, 4, 4096
REP = (1 << 32) // (P * H) + 1  # T * H just past 2^32; T * K * I past it too


@pytest.mark.emu_skip("needs tens of GiB of buffers and queries free device memory")
def test_offsets_past_32_bits(dev, tsm):
    need = 80 << 30
    free, _ = torch.cuda.mem_get_info()
    if free < need:
        pytest.skip(f"needs {need >> 30} GiB of free device memory, {free >> 30} GiB free")
    T = REP * P
    assert T * H >= 1 << 32 and T * K * I >= 1 << 32 and T < 1 << 24
    print(f"large batch T={T} H={H} I={I} E={E} k={K}", flush=True)
    x, gw, w13, w2 = make_layer(P, H, E, I, torch.bfloat16, seed=77, device=dev)
    p13, p2 = tsm.pack_moe_weights(w13, w2)
    w, ids, _ = tsm.moe_router(x, gw, K, True)
    small = tsm.fused_moe_packed(x, p13, p2, w, ids)

    xb = x.repeat(REP, 1)
    wb, idsb, _ = tsm.moe_router(xb, gw, K, True)
    # the router is row-wise too
    assert torch.equal(idsb.view(REP, P, K)[-1], ids) and torch.equal(wb.view(REP, P, K)[-1], w)
    big = tsm.fused_moe_packed(xb, p13, p2, wb, idsb)
    torch.cuda.synchronize()
    del xb, wb, idsb
    bv = big.view(REP, P, H)
    for r0 in range(0, REP, 64):
        chunk = bv[r0:r0 + 64]
        bad = (chunk != small.unsqueeze(0)).flatten(1).any(1)
        assert not bad.any(), f"period {r0 + int(bad.nonzero()[0])} differs from the first"
