"""Torch-CPU restatement of the reference's attention-side math (TEST INFRASTRUCTURE ONLY).

Only tests/ may import this module, and only as the checker; the product package never does.

Functions and the reference code they restate:
- rms_norm_ref          serve.py:799-809  RMSNorm in fp32, cast back to the input dtype.
- rotary_ref            serve.py:811-814  rotate-half RoPE in fp32 on [x1 | x2] halves.
- qk_norm_rope_ref      serve.py:868-879  per-head q/k RMSNorm (Qwen3) then RoPE.
- paged_attention_ref   serve.py:639-688  torch_ref_attention: per request, gather the live
                                          pages, expand the KV heads for GQA, causal SDPA with
                                          the queries at the last q_len positions.
- dense_attention_fp64  textbook softmax(q k^T * scale + causal mask) v per (token, head) in
                        float64, used only to pin paged_attention_ref.
The K and V caches here are in the reference's layout, [num_pages, page, Hkv, D]; tests build
the build's transposed V pages from the same values.
"""
import torch
import torch.nn.functional as F


def rms_norm_ref(x, weight, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)


def rotary_ref(x, cos, sin):
    """x [T, heads, D]; cos/sin [T, D/2] fp32."""
    x1, x2 = x.float().chunk(2, dim=-1)
    cos, sin = cos[:, None], sin[:, None]
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1).to(x.dtype)


def qk_norm_rope_ref(q, k, cos, sin, q_weight=None, k_weight=None, eps=1e-6):
    if q_weight is not None:
        q, k = rms_norm_ref(q, q_weight, eps), rms_norm_ref(k, k_weight, eps)
    return rotary_ref(q, cos, sin), rotary_ref(k, cos, sin)


def paged_attention_ref(q, k_cache, v_cache, query_start_loc, seq_lens, block_table, scale):
    """q [T, H, D]; caches [num_pages, page, Hkv, D]; query_start_loc (list, B+1); seq_lens
    (list, B: context length after this step); block_table [B, max_pages]."""
    out = torch.empty_like(q)
    H, Hkv, bs = q.shape[1], k_cache.shape[2], k_cache.shape[1]
    for i in range(len(seq_lens)):
        s, e, kv_len = query_start_loc[i], query_start_loc[i + 1], seq_lens[i]
        q_len = e - s
        if q_len == 0:
            continue
        blocks = block_table[i, : -(-kv_len // bs)].long()
        k = k_cache[blocks].flatten(0, 1)[:kv_len]
        v = v_cache[blocks].flatten(0, 1)[:kv_len]
        k = k.transpose(0, 1).repeat_interleave(H // Hkv, 0)
        v = v.transpose(0, 1).repeat_interleave(H // Hkv, 0)
        q_pos = torch.arange(kv_len - q_len, kv_len)
        mask = torch.arange(kv_len)[None, :] <= q_pos[:, None]
        o = F.scaled_dot_product_attention(q[s:e].transpose(0, 1), k, v, attn_mask=mask,
                                           scale=scale)
        out[s:e] = o.transpose(0, 1)
    return out


def dense_attention_fp64(q, keys, values, scale):
    """One request: q [q_len, H, D], keys/values [kv_len, Hkv, D] in context order."""
    q_len, H, D = q.shape
    kv_len, Hkv, _ = keys.shape
    out = torch.zeros(q_len, H, D, dtype=torch.float64)
    for t in range(q_len):
        pos = kv_len - q_len + t
        for h in range(H):
            kh = h // (H // Hkv)
            s = (keys[: pos + 1, kh].double() @ q[t, h].double()) * scale
            p = torch.softmax(s, 0)
            out[t, h] = p @ values[: pos + 1, kh].double()
    return out
