"""The MFMA-tiled ("packed") expert-weight layout as tensor permutations.

packed[e][blk][s][lane][i] = W[e][16*src(blk) + lane%16][32*s + 8*(lane//16) + i]

with src(blk) = blk for w2 ([E, H, I]) and, for w13 ([E, 2I, H]), src(2j) = j (gate rows) and
src(2j+1) = I/16 + j (the matching up rows). Padded shapes (ops.padded_shape) place W in the
top-left corner of a zero [N_pad, K_pad] matrix per expert (per half, for w13) first.

The HIP kernel behind ops.pack_moe_weights produces this layout on the GPU at load time; these
functions are its inverse (`unpack`, used when a module hands its weights back in the reference
layout: state_dict, checkpoint loading) and a device-independent statement of the same layout
(`pack`), which the CPU tests compare against an element-by-element reading of the formula.
"""
import torch
from torch import Tensor


def _pad(w: Tensor, n_pad: int, k_pad: int) -> Tensor:
    E, N, K = w.shape
    if (N, K) == (n_pad, k_pad):
        return w
    out = w.new_zeros(E, n_pad, k_pad)
    out[:, :N, :K] = w
    return out


def pack(w: Tensor, interleave: bool, n_pad: int = None, k_pad: int = None) -> Tensor:
    """Packed copy of w [E, N, K] (w13 with interleave=True, N = 2I; w2 with interleave=False),
    padded to [E, n_pad, k_pad] (n_pad = 2 I_pad for w13)."""
    E, N, K = w.shape
    n_pad = N if n_pad is None else n_pad
    k_pad = K if k_pad is None else k_pad
    if n_pad % (32 if interleave else 16) or k_pad % 32:
        raise ValueError(f"packed shape [{n_pad}, {k_pad}] is not a multiple of the MFMA blocks")
    ks = k_pad // 32
    if interleave:
        half, half_pad = N // 2, n_pad // 2
        wp = torch.cat([_pad(w[:, :half], half_pad, k_pad), _pad(w[:, half:], half_pad, k_pad)],
                       dim=1)
        # (e, half, j, r, s, q, i) -> (e, j, half, s, q, r, i): block 2j + half
        v = wp.reshape(E, 2, half_pad // 16, 16, ks, 4, 8).permute(0, 2, 1, 4, 5, 3, 6)
    else:
        wp = _pad(w, n_pad, k_pad)
        # (e, blk, r, s, q, i) -> (e, blk, s, q, r, i)
        v = wp.reshape(E, n_pad // 16, 16, ks, 4, 8).permute(0, 1, 3, 4, 2, 5)
    return v.contiguous().reshape(E, n_pad, k_pad)


def unpack(p: Tensor, interleave: bool, n: int = None, k: int = None) -> Tensor:
    """Reference-layout [E, n, k] weights from a packed [E, n_pad, k_pad] tensor (inverse of
    `pack`; n = 2I for w13)."""
    E, n_pad, k_pad = p.shape
    n = n_pad if n is None else n
    k = k_pad if k is None else k
    ks = k_pad // 32
    if interleave:
        half_pad, half = n_pad // 2, n // 2
        v = p.reshape(E, half_pad // 16, 2, ks, 4, 16, 8).permute(0, 2, 1, 5, 3, 4, 6)
        w = v.contiguous().reshape(E, 2, half_pad, k_pad)[:, :, :half, :k]
        return w.reshape(E, n, k).contiguous()
    v = p.reshape(E, n_pad // 16, ks, 4, 16, 8).permute(0, 1, 4, 2, 3, 5)
    return v.contiguous().reshape(E, n_pad, k_pad)[:, :n, :k].contiguous()
