"""CPU pinning of the attention-side oracle (oracle/attn_oracle.py), which restates serve.py's
RMSNorm, rotary and torch_ref_attention: against float64 textbook formulas, closed forms and
known answers."""
import math

import torch

from oracle.attn_oracle import (dense_attention_fp64, paged_attention_ref, qk_norm_rope_ref,
                                rms_norm_ref, rotary_ref)


def test_rms_norm_ref_against_fp64():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 3, 64, generator=g).bfloat16()
    w = (1 + 0.1 * torch.randn(64, generator=g)).bfloat16()
    out = rms_norm_ref(x, w, 1e-6).double()
    xd = x.double()
    ref = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert (out - ref).abs().max() <= (ref.abs() * 2.0 ** -7).max()


def test_rotary_ref_is_a_rotation():
    """cos = 1, sin = 0 is the identity; each pair (x_j, x_{j+D/2}) is rotated by its angle:
    norms are kept, and rotating by -angle undoes it (fp32 inputs, so no bf16 rounding)."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 2, 16, generator=g)
    ang = torch.rand(4, 8, generator=g) * 6.0
    ident = rotary_ref(x, torch.ones(4, 8), torch.zeros(4, 8))
    assert torch.equal(ident, x)
    y = rotary_ref(x, ang.cos(), ang.sin())
    n0 = x[..., :8] ** 2 + x[..., 8:] ** 2
    n1 = y[..., :8] ** 2 + y[..., 8:] ** 2
    assert torch.allclose(n0, n1, atol=1e-5)
    back = rotary_ref(y, ang.cos(), -ang.sin())
    assert torch.allclose(back, x, atol=1e-5)
    # quarter turn: (x1, x2) -> (-x2, x1)
    q = rotary_ref(x, torch.zeros(4, 8), torch.ones(4, 8))
    assert torch.equal(q, torch.cat([-x[..., 8:], x[..., :8]], -1))


def test_qk_norm_rope_ref_order():
    """Norm first, then the rotation (a rotation keeps the per-head norm, so the normed
    rotated head has unit rms times the weight only when the weight is uniform)."""
    g = torch.Generator().manual_seed(2)
    q = torch.randn(3, 4, 32, generator=g) * 5
    k = torch.randn(3, 2, 32, generator=g) * 5
    ang = torch.rand(3, 16, generator=g)
    w = torch.full((32,), 2.0)
    qo, ko = qk_norm_rope_ref(q, k, ang.cos(), ang.sin(), w, w, 0.0)
    assert torch.allclose(qo.pow(2).mean(-1), torch.full((3, 4), 4.0), atol=1e-4)
    assert torch.allclose(ko.pow(2).mean(-1), torch.full((3, 2), 4.0), atol=1e-4)


def _pack_request_pages(keys_list, values_list, page, num_pages, gen):
    """Scatter each request's K/V into random distinct pages; returns caches and block table."""
    Hkv, D = keys_list[0].shape[1:]
    kc = torch.randn(num_pages, page, Hkv, D, generator=gen) * 100   # garbage elsewhere
    vc = torch.randn(num_pages, page, Hkv, D, generator=gen) * 100
    perm = torch.randperm(num_pages - 1, generator=gen) + 1
    maxp = max(-(-k.shape[0] // page) for k in keys_list)
    bt = torch.zeros(len(keys_list), maxp, dtype=torch.int32)
    nxt = 0
    for b, (k, v) in enumerate(zip(keys_list, values_list)):
        n = -(-k.shape[0] // page)
        for j in range(n):
            pg = int(perm[nxt]); nxt += 1
            bt[b, j] = pg
            seg = slice(j * page, min((j + 1) * page, k.shape[0]))
            kc[pg, : seg.stop - seg.start] = k[seg]
            vc[pg, : seg.stop - seg.start] = v[seg]
    return kc, vc, bt


def test_paged_attention_ref_against_dense_fp64():
    g = torch.Generator().manual_seed(3)
    H, Hkv, D, page = 4, 2, 16, 4
    q_lens, kv_lens = [3, 1, 5, 0], [7, 9, 5, 0]
    keys = [torch.randn(n, Hkv, D, generator=g) for n in kv_lens]
    vals = [torch.randn(n, Hkv, D, generator=g) for n in kv_lens]
    kc, vc, bt = _pack_request_pages(keys[:3], vals[:3], page, 16, g)
    bt = torch.cat([bt, torch.zeros(1, bt.shape[1], dtype=torch.int32)])
    qsl = [0]
    for n in q_lens:
        qsl.append(qsl[-1] + n)
    q = torch.randn(qsl[-1], H, D, generator=g)
    scale = D ** -0.5
    out = paged_attention_ref(q, kc, vc, qsl, kv_lens, bt, scale)
    for b in range(3):
        ref = dense_attention_fp64(q[qsl[b]:qsl[b + 1]], keys[b], vals[b], scale)
        assert torch.allclose(out[qsl[b]:qsl[b + 1]].double(), ref, atol=1e-5), b


def test_attention_known_answers():
    """A query that sees a single key returns that key's value; equal scores average the
    values; a large score gap selects the top key's value."""
    D = 8
    keys = torch.zeros(3, 1, D)
    vals = torch.arange(3 * D, dtype=torch.float32).view(3, 1, D)
    q = torch.zeros(3, 1, D)
    out = dense_attention_fp64(q, keys, vals, 1.0)   # positions 0, 1, 2 (causal)
    assert torch.allclose(out[0, 0], vals[0, 0].double())
    assert torch.allclose(out[2, 0], vals.double().mean(0)[0])
    keys[1, 0, 0] = 1.0
    q2 = torch.zeros(1, 1, D)
    q2[0, 0, 0] = 1000.0
    out2 = dense_attention_fp64(q2, keys[:2], vals[:2], 1.0)
    assert torch.allclose(out2[0, 0], vals[1, 0].double())
    assert math.isclose(float(out2.sum()), float(vals[1].sum()), rel_tol=1e-9)
