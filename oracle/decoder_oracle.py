"""Torch-CPU restatement of serve.py's qwen3_moe decoder forward (TEST INFRASTRUCTURE ONLY).

Only tests/ may import this module, and only as the checker; the product package never does.

decoder_reference restates Model.forward / DecoderLayer.forward with the torch (non-Triton)
branches of serve.py: add_rmsnorm (serve.py:1185-1193: residual = residual + x, then RMSNorm),
Attention.project / attend (serve.py:839-906: fused qkv Linear, per-head q/k RMSNorm, rotary,
causal attention over the sequence), SparseMoE.forward's torch path (serve.py:1089-1099: router,
softmax, top-k, renormalise, moe_reference), the final add_rmsnorm and the LM head
(serve.py:1254-1263). The RoPE table is built as serve.py:1240-1247 builds it.
The router takes fp32 logits here (F.linear of the fp32-cast inputs), the definition the tests
pin the build's router to; serve.py's bf16 Linear rounds them to bf16 first.

It takes a flat state dict with the driver's parameter names and dense [B, S] token ids (every
sequence attends to its own prefix; no paging, which the attention oracle covers).
"""
import torch
import torch.nn.functional as F

from .attn_oracle import rms_norm_ref, rotary_ref
from .moe_oracle import moe_reference, route_torch


def rope_table(D, theta, n):
    inv = 1.0 / theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D)
    freqs = torch.outer(torch.arange(n, dtype=torch.float64), inv)
    return freqs.cos().float(), freqs.sin().float()


def decoder_reference(sd, cfg, ids, return_route_gaps=False):
    """sd: parameter name -> CPU tensor (bf16); ids [B, S]. Returns logits [B, S, vocab] fp32;
    with return_route_gaps, also [B, S]: per position, the smallest gap over the layers between
    the k-th and the (k+1)-th routing probability (a near tie there can route differently under
    any other summation order, so a comparison should not rely on such positions)."""
    B, S = ids.shape
    H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps, k = cfg.rms_norm_eps, cfg.num_experts_per_tok
    cos, sin = rope_table(D, cfg.rope_theta, S)
    out, gaps = [], []
    for b in range(B):
        gap = torch.full((S,), float("inf"))
        x = sd["embed.weight"][ids[b]]                      # [S, hidden] bf16
        residual = None
        for L in range(cfg.num_hidden_layers):
            p = f"layers.{L}."
            residual = x if residual is None else residual + x
            h = rms_norm_ref(residual, sd[p + "input_norm"], eps)
            qkv = h @ sd[p + "attn.qkv_proj.weight"].t()
            q, kk, v = qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
            q, kk, v = q.reshape(S, H, D), kk.reshape(S, Hkv, D), v.reshape(S, Hkv, D)
            q = rotary_ref(rms_norm_ref(q, sd[p + "attn.q_norm"], eps), cos, sin)
            kk = rotary_ref(rms_norm_ref(kk, sd[p + "attn.k_norm"], eps), cos, sin)
            kx = kk.transpose(0, 1).repeat_interleave(H // Hkv, 0)
            vx = v.transpose(0, 1).repeat_interleave(H // Hkv, 0)
            o = F.scaled_dot_product_attention(q.transpose(0, 1), kx, vx, is_causal=True,
                                               scale=D ** -0.5).transpose(0, 1)
            a = o.reshape(S, H * D) @ sd[p + "attn.o_proj.weight"].t()
            residual = residual + a
            h = rms_norm_ref(residual, sd[p + "post_attn_norm"], eps)
            logits = F.linear(h.float(), sd[p + "mlp.gate.weight"].float())
            w, e = route_torch(logits, k, cfg.norm_topk_prob)
            srt = logits.softmax(-1).sort(-1, descending=True).values
            if k < srt.shape[-1]:
                gap = torch.minimum(gap, srt[:, k - 1] - srt[:, k])
            x = moe_reference(h, sd[p + "mlp.w13"], sd[p + "mlp.w2"], w, e)
        residual = residual + x
        h = rms_norm_ref(residual, sd["norm"], eps)
        out.append((h @ sd["lm_head.weight"].t()).float())
        gaps.append(gap)
    if return_route_gaps:
        return torch.stack(out), torch.stack(gaps)
    return torch.stack(out)
