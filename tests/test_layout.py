"""The packed expert-weight layout as tensor permutations (tinyserve_amd/layout.py), checked on the
CPU against an element-by-element reading of its definition
    packed[e][blk][s][lane][i] = W[e][16*src(blk) + lane%16][32*s + 8*(lane//16) + i]
(src(2j) = j, src(2j+1) = I_pad/16 + j for w13; zero outside W), including padded shapes, and the
inverse used to hand weights back in the reference layout."""
import numpy as np
import pytest
import torch

from tinyserve_amd import layout


def packed_by_definition(W, interleave, n_pad, k_pad):
    E, N, K = W.shape
    out = np.zeros((E, n_pad, k_pad), dtype=W.dtype)
    flat = out.reshape(E, n_pad // 16, k_pad // 32, 64, 8)
    half, half_pad = N // 2, n_pad // 2
    for e in range(E):
        for blk in range(n_pad // 16):
            for s in range(k_pad // 32):
                for lane in range(64):
                    for i in range(8):
                        r, k = lane % 16, 32 * s + 8 * (lane // 16) + i
                        if interleave:
                            h, row = blk & 1, 16 * (blk >> 1) + r
                            ok = row < half and k < K
                            src = h * half + row
                        else:
                            row = 16 * blk + r
                            ok = row < N and k < K
                            src = row
                        if ok:
                            flat[e, blk, s, lane, i] = W[e, src, k]
    return out


@pytest.mark.parametrize("interleave,N,K,n_pad,k_pad", [
    (True, 64, 64, 64, 64),      # w13 with I = 32, H = 64
    (False, 32, 64, 32, 64),     # w2
    (True, 2 * 24, 40, 64, 64),  # ragged I = 24 (pads to 32 per half) and K = 40
    (False, 40, 24, 48, 32),     # ragged H = 40, I = 24
])
def test_pack_matches_definition_and_inverts(interleave, N, K, n_pad, k_pad):
    g = torch.Generator().manual_seed(N * 1000 + K)
    W = torch.randn(2, N, K, generator=g)
    P = layout.pack(W, interleave, n_pad, k_pad)
    ref = packed_by_definition(W.numpy(), interleave, n_pad, k_pad)
    assert np.array_equal(P.numpy(), ref)
    assert torch.equal(layout.unpack(P, interleave, N, K), W)


def test_unpadded_pack_is_a_permutation():
    W = torch.arange(2 * 64 * 64, dtype=torch.float32).reshape(2, 64, 64)
    P = layout.pack(W, True)
    assert P.shape == W.shape
    assert torch.equal(torch.sort(P.flatten()).values, W.flatten())
