"""Minimal qwen3_moe model driver: the end-to-end workload around the MoE op.

A random-init Qwen3-MoE decoder (the architecture of serve.py's qwen3_moe path: pre-norm
residual blocks, GQA attention with per-head q/k RMSNorm and rotary embeddings, a SparseMoE
feed-forward in every layer, final norm and LM head, serve.py:1100-1258) run as batched greedy
generation: all prompts prefilled in one pass, then one token per sequence per step against a
contiguous KV cache. Attention, norms and projections are stock PyTorch (SDPA, hipBLASLt GEMMs);
every MoE block is `tinyserve_amd.SparseMoE` on the HIP kernels. This is a workload driver for
measuring the op inside a model, not a serving engine: no paged KV cache, scheduler, sampling or
tokenizer (prompts are synthetic token ids).
"""
import time
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from .moe import SparseMoE


@dataclass
class Qwen3MoeConfig:
    """Qwen3-30B-A3B shape by default."""
    hidden_size: int = 2048
    num_hidden_layers: int = 48
    num_attention_heads: int = 32
    num_key_value_heads: int = 4
    head_dim: int = 128
    vocab_size: int = 151936
    num_experts: int = 128
    num_experts_per_tok: int = 8
    moe_intermediate_size: int = 768
    norm_topk_prob: bool = True
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6


def rms_norm(x, weight, eps):
    """RMSNorm in fp32, weight applied after casting back (as HF Qwen3RMSNorm)."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * xf.to(x.dtype)


def rotary(x, cos, sin):
    """Rotate-half rotary embedding; x [..., S, D], cos/sin [S, D]."""
    h = x.shape[-1] // 2
    rot = torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    return x * cos + rot * sin


class Attention(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.nh, self.nkv, self.d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        H = cfg.hidden_size
        self.qkv_proj = nn.Linear(H, (self.nh + 2 * self.nkv) * self.d, bias=False)
        self.o_proj = nn.Linear(self.nh * self.d, H, bias=False)
        self.q_norm = nn.Parameter(torch.ones(self.d))
        self.k_norm = nn.Parameter(torch.ones(self.d))
        self.eps = cfg.rms_norm_eps

    def forward(self, x, cos, sin, cache_k, cache_v, start):
        B, S, _ = x.shape
        q, k, v = self.qkv_proj(x).split(
            [self.nh * self.d, self.nkv * self.d, self.nkv * self.d], dim=-1)
        q = rms_norm(q.view(B, S, self.nh, self.d), self.q_norm, self.eps).transpose(1, 2)
        k = rms_norm(k.view(B, S, self.nkv, self.d), self.k_norm, self.eps).transpose(1, 2)
        v = v.view(B, S, self.nkv, self.d).transpose(1, 2)
        q, k = rotary(q, cos, sin), rotary(k, cos, sin)
        cache_k[:, :, start:start + S] = k
        cache_v[:, :, start:start + S] = v
        kk, vv = cache_k[:, :, :start + S], cache_v[:, :, :start + S]
        # prefill (start 0): causal within the prompt; decode (S = 1): the whole cache
        o = F.scaled_dot_product_attention(q, kk, vv, is_causal=S > 1, enable_gqa=True)
        return self.o_proj(o.transpose(1, 2).reshape(B, S, self.nh * self.d))

    def decode(self, x, cos, sin, cache_k, cache_v, pos, mask):
        """One token per sequence at position `pos` (a device tensor), attending over the whole
        fixed-length cache under `mask`: shapes and addresses never change, so a step can be
        captured once in a HIP graph and replayed."""
        B = x.shape[0]
        q, k, v = self.qkv_proj(x).split(
            [self.nh * self.d, self.nkv * self.d, self.nkv * self.d], dim=-1)
        q = rms_norm(q.view(B, 1, self.nh, self.d), self.q_norm, self.eps).transpose(1, 2)
        k = rms_norm(k.view(B, 1, self.nkv, self.d), self.k_norm, self.eps).transpose(1, 2)
        v = v.view(B, 1, self.nkv, self.d).transpose(1, 2)
        q, k = rotary(q, cos, sin), rotary(k, cos, sin)
        cache_k.index_copy_(2, pos, k)
        cache_v.index_copy_(2, pos, v)
        # query heads grouped per kv head (head h reads kv head h // (nh / nkv), as SDPA's
        # enable_gqa does): two batched matmuls over the cache, no K/V expansion
        qg = q.reshape(B, self.nkv, self.nh // self.nkv, self.d)
        s = torch.matmul(qg, cache_k.transpose(-1, -2)).float() * (self.d ** -0.5)
        s = s.masked_fill(~mask, float("-inf"))
        o = torch.matmul(torch.softmax(s, dim=-1).to(x.dtype), cache_v)  # [B, nkv, G, d]
        return self.o_proj(o.reshape(B, 1, self.nh * self.d))


class DecoderLayer(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.input_norm = nn.Parameter(torch.ones(cfg.hidden_size))
        self.post_attn_norm = nn.Parameter(torch.ones(cfg.hidden_size))
        self.attn = Attention(cfg)
        self.mlp = SparseMoE(cfg)
        self.eps = cfg.rms_norm_eps

    def forward(self, x, cos, sin, cache_k, cache_v, start):
        x = x + self.attn(rms_norm(x, self.input_norm, self.eps), cos, sin, cache_k, cache_v,
                          start)
        B, S, H = x.shape
        h = rms_norm(x, self.post_attn_norm, self.eps).reshape(B * S, H)
        return x + self.mlp(h).view(B, S, H)

    def decode(self, x, cos, sin, cache_k, cache_v, pos, mask):
        x = x + self.attn.decode(rms_norm(x, self.input_norm, self.eps), cos, sin, cache_k,
                                 cache_v, pos, mask)
        B, _, H = x.shape
        return x + self.mlp(rms_norm(x, self.post_attn_norm, self.eps).reshape(B, H)).view(B, 1, H)


class Qwen3MoeModel(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(cfg) for _ in range(cfg.num_hidden_layers))
        self.norm = nn.Parameter(torch.ones(cfg.hidden_size))
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2).float() / cfg.head_dim))
        self.register_buffer("inv_freq", inv, persistent=False)

    @torch.no_grad()
    def init_random(self, seed=0, std=0.02):
        """Random-init weights (N(0, std) matrices, unit norms) in place."""
        g = torch.Generator(device=self.norm.device).manual_seed(seed)
        for name, p in self.named_parameters():
            if p.dim() >= 2:
                p.normal_(0.0, std, generator=g)
            else:
                p.fill_(1.0)
        for layer in self.layers:
            layer.mlp.pack()

    def rope(self, start, S, device, dtype):
        pos = torch.arange(start, start + S, device=device, dtype=torch.float32)
        f = torch.outer(pos, self.inv_freq.to(device))
        emb = torch.cat((f, f), dim=-1)
        return emb.cos().to(dtype), emb.sin().to(dtype)

    def new_cache(self, batch, max_len):
        # zero-filled: masked positions take weight 0 in attention, and 0 * garbage could be NaN
        c = self.cfg
        shape = (batch, c.num_key_value_heads, max_len, c.head_dim)
        dev, dt = self.norm.device, self.norm.dtype
        return [(torch.zeros(shape, device=dev, dtype=dt), torch.zeros(shape, device=dev, dtype=dt))
                for _ in range(c.num_hidden_layers)]

    @torch.no_grad()
    def forward(self, ids, cache, start, last_only=True):
        x = self.embed(ids)
        cos, sin = self.rope(start, ids.shape[1], x.device, x.dtype)
        for layer, (ck, cv) in zip(self.layers, cache):
            x = layer(x, cos, sin, ck, cv, start)
        if last_only:
            x = x[:, -1:]
        return self.lm_head(rms_norm(x, self.norm, self.cfg.rms_norm_eps)).float()

    @torch.no_grad()
    def decode_step(self, tok, cache, pos):
        """tok [B, 1] at position pos (int64 device tensor [1]) -> logits [B, vocab] fp32."""
        x = self.embed(tok)
        f = pos.float()[:, None] * self.inv_freq[None, :]
        emb = torch.cat((f, f), dim=-1)
        cos, sin = emb.cos().to(x.dtype), emb.sin().to(x.dtype)
        L = cache[0][0].shape[2]
        mask = (torch.arange(L, device=x.device) <= pos)[None, None, None, :]  # [1,1,1,L]
        for layer, (ck, cv) in zip(self.layers, cache):
            x = layer.decode(x, cos, sin, ck, cv, pos, mask)
        return self.lm_head(rms_norm(x[:, 0], self.norm, self.cfg.rms_norm_eps)).float()


@torch.no_grad()
def generate(model, prompts, new_tokens, graph=True):
    """Greedy generation for a batch of equal-length prompts [B, P]. Returns (tokens [B, N],
    prefill seconds, decode seconds). The prompts are prefilled in one pass; each decode step
    runs on the fixed-length cache, captured once as a HIP graph and replayed (graph=True), as
    serve.py replays captured decode steps, or eagerly."""
    B, P = prompts.shape
    cache = model.new_cache(B, P + new_tokens)
    out = torch.empty(B, new_tokens, dtype=torch.long, device=prompts.device)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out[:, 0] = model(prompts, cache, 0)[:, -1].argmax(-1)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    tok = out[:, :1].clone()
    pos = torch.full((1,), P, dtype=torch.long, device=prompts.device)
    col = torch.ones(1, dtype=torch.long, device=prompts.device)

    def step():
        nxt = model.decode_step(tok, cache, pos).argmax(-1, keepdim=True)
        out.index_copy_(1, col, nxt)
        tok.copy_(nxt)
        pos.add_(1)
        col.add_(1)

    if graph and new_tokens > 1:
        # warm up on a side stream (kernels, allocator), then capture one step; the warm-up
        # advanced the state, so rewind it before replaying
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        tok.copy_(out[:, :1])
        pos.fill_(P)
        col.fill_(1)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(new_tokens - 1):
            g.replay()
    else:
        for _ in range(new_tokens - 1):
            step()
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    return out, t1 - t0, t2 - t1


def build_model(cfg=None, device="cuda", seed=0):
    cfg = cfg or Qwen3MoeConfig()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen3MoeModel(cfg)
    finally:
        torch.set_default_dtype(torch.float32)
    model.init_random(seed)
    return model


def run_e2e(batch=64, prompt_len=512, new_tokens=256, cfg=None, seed=0):
    """Config 5 of the benchmark set: returns a dict of timings and throughputs."""
    model = build_model(cfg, seed=seed)
    g = torch.Generator(device="cuda").manual_seed(seed + 1)
    prompts = torch.randint(0, model.cfg.vocab_size, (batch, prompt_len), device="cuda",
                            generator=g)
    generate(model, prompts[:, :16], 4)  # warm-up (kernels, allocator)
    toks, tp, td = generate(model, prompts, new_tokens)
    return {"batch": batch, "prompt_len": prompt_len, "new_tokens": new_tokens,
            "layers": model.cfg.num_hidden_layers,
            "prefill_s": tp, "prefill_tokens_per_s": batch * prompt_len / tp,
            "decode_s": td, "decode_tokens_per_s": batch * (new_tokens - 1) / td,
            "decode_ms_per_step": td / max(new_tokens - 1, 1) * 1e3,
            "first_tokens": toks[0, :8].tolist()}
