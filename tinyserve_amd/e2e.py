"""Minimal qwen3_moe model driver: the end-to-end workload around the MoE op.

A random-init Qwen3-MoE decoder with the structure of serve.py's Model / DecoderLayer
(serve.py:1100-1258): residual stream carried between layers and added inside the norms
(add_rmsnorm, serve.py:1185-1193), GQA attention with per-head q/k RMSNorm and rotary embeddings
over a paged KV cache (serve.py:816-906), a SparseMoE feed-forward in every layer, final norm and
LM head. Everything but the dense projections runs on this build's HIP kernels:
    embedding / qkv_proj / o_proj / lm_head   torch (hipBLASLt GEMMs)
    input norm + residual add                 ops.rmsnorm / ops.moe_combine_add_rmsnorm
    q/k norm + RoPE + K/V page write          attention.qk_norm_rope
    paged causal attention                    attention.paged_attention
    MoE block                                 SparseMoE (router + experts), per-slot rows
    MoE k-sum + next residual add + norm      ops.moe_combine_add_rmsnorm (one launch)
    greedy token                              attention.greedy_argmax
Requests are packed back to back (serve.py's flattened batch, AttnMetadata serve.py:627-637);
`generate` prefills the prompts and then decodes one token per sequence per step, each decode
step replayed from one captured HIP graph. It is a workload driver for measuring the op inside a
model, not a serving engine: no scheduler, sampling or tokenizer (prompts are synthetic ids).
"""
import time
from dataclasses import dataclass
from types import SimpleNamespace

import torch
import torch.nn.functional as F
from torch import nn

from . import ops
from .attention import PagedKVCache, greedy_argmax, paged_attention, qk_norm_rope
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


class Attention(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.H, self.Hkv, self.D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.qkv_sizes = [self.H * self.D, self.Hkv * self.D, self.Hkv * self.D]
        self.qkv_proj = nn.Linear(cfg.hidden_size, sum(self.qkv_sizes), bias=False)
        self.o_proj = nn.Linear(self.H * self.D, cfg.hidden_size, bias=False)
        self.q_norm = nn.Parameter(torch.ones(self.D))
        self.k_norm = nn.Parameter(torch.ones(self.D))
        self.eps = cfg.rms_norm_eps

    def forward(self, x, cos, sin, cache: PagedKVCache, meta):
        T = x.shape[0]
        q, k, v = self.qkv_proj(x).split(self.qkv_sizes, dim=-1)
        q, k, v = q.view(T, self.H, self.D), k.view(T, self.Hkv, self.D), v.view(T, self.Hkv, self.D)
        qk_norm_rope(q, k, cos, sin, self.q_norm, self.k_norm, self.eps, v, cache.k, cache.v,
                     meta.slot_mapping)
        o = paged_attention(q, cache.k, cache.v, meta, self.D ** -0.5)
        return self.o_proj(o.view(T, self.H * self.D))


class DecoderLayer(nn.Module):
    def __init__(self, cfg, router_logits="model"):
        super().__init__()
        self.input_norm = nn.Parameter(torch.ones(cfg.hidden_size))
        self.post_attn_norm = nn.Parameter(torch.ones(cfg.hidden_size))
        self.attn = Attention(cfg)
        self.mlp = SparseMoE(cfg, router_logits=router_logits)
        self.eps = cfg.rms_norm_eps

    def forward(self, x, residual, cos, sin, cache, meta):
        """(x, residual) -> (MoE per-slot rows, residual), the reference's layer convention
        (serve.py:1177-1183) with the MoE output left unsummed: the next norm sums it.
        x is the previous layer's rows [T*k, H] (or the embeddings, for the first layer, with
        residual None)."""
        if residual is None:
            h = ops.rmsnorm(x, self.input_norm, self.eps)
            residual = x
        else:
            h = ops.moe_combine_add_rmsnorm(x, self.mlp.top_k, residual, self.input_norm,
                                            self.eps)
        a = self.attn(h, cos, sin, cache, meta)
        h = ops.rmsnorm(a, self.post_attn_norm, self.eps, residual)
        return self.mlp.rows(h), residual


class Qwen3MoeModel(nn.Module):
    def __init__(self, cfg, max_position=4096, router_logits="model"):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(cfg, router_logits)
                                    for _ in range(cfg.num_hidden_layers))
        self.norm = nn.Parameter(torch.ones(cfg.hidden_size))
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        D = cfg.head_dim
        inv = 1.0 / cfg.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D)
        freqs = torch.outer(torch.arange(max_position, dtype=torch.float64), inv)
        self.register_buffer("cos", freqs.cos().float(), persistent=False)
        self.register_buffer("sin", freqs.sin().float(), persistent=False)

    @torch.no_grad()
    def init_random(self, seed=0, std=0.02):
        """Random-init weights (N(0, std) matrices, unit norms) in place, then pack the experts."""
        g = torch.Generator(device=self.norm.device).manual_seed(seed)
        for name, p in self.named_parameters():
            if p.dim() >= 2:
                p.normal_(0.0, std, generator=g)
            else:
                p.fill_(1.0)
        for layer in self.layers:
            layer.mlp.pack()

    @torch.inference_mode()
    def autotune(self, max_num_tokens, reps=5):
        """Time the expert plans per batch-size bucket and install the fastest, as the reference
        engine does at start-up before capturing graphs (serve.py:1692-1705: autotune_fused_moe
        on the first layer's weights; every layer has the same shapes). Returns the table."""
        from .kernels import autotune_fused_moe
        mlp = self.layers[0].mlp
        w13, w2 = mlp.pack() if mlp.packed else (mlp.w13, mlp.w2)
        return autotune_fused_moe(w13, w2, mlp.top_k, max_num_tokens, packed=mlp.packed,
                                  reps=reps)

    def new_caches(self, num_pages, page=16):
        c = self.cfg
        return [PagedKVCache.allocate(num_pages, page, c.num_key_value_heads, c.head_dim,
                                      self.norm.device, self.norm.dtype)
                for _ in range(c.num_hidden_layers)]

    @torch.no_grad()
    def forward(self, ids, positions, meta, caches, last_rows):
        """ids / positions [T] (packed requests), meta as serve.AttnMetadata, last_rows [B]:
        the packed row of each request's last token. Returns logits [B, vocab] (fp32)."""
        x = self.embed(ids)
        cos, sin = self.cos[positions], self.sin[positions]
        residual = None
        for layer, cache in zip(self.layers, caches):
            x, residual = layer(x, residual, cos, sin, cache, meta)
        h = ops.moe_combine_add_rmsnorm(x, self.cfg.num_experts_per_tok, residual, self.norm,
                                        self.cfg.rms_norm_eps)
        return self.lm_head(h[last_rows]).float()


class PagedBatch:
    """Page assignment and device metadata for B sequences of up to max_len tokens: sequence b
    owns pages 1 + b * pps .. (page 0 is the null page), so its block table row is fixed."""

    def __init__(self, B, max_len, page, device):
        self.B, self.page = B, page
        self.pps = -(-max_len // page)
        self.num_pages = 1 + B * self.pps
        self.block_table = (1 + torch.arange(B * self.pps, dtype=torch.int32, device=device)
                            ).view(B, self.pps)
        self.device = device

    def slots(self, seq, pos):
        """Cache slot of token position `pos` of sequence `seq` (device tensors)."""
        pg = self.block_table[seq, torch.div(pos, self.page, rounding_mode="floor")].long()
        return pg * self.page + pos % self.page

    def prefill_meta(self, lens):
        """Metadata for prompts of lengths `lens` (list) packed back to back, from position 0."""
        dev = self.device
        qsl = [0]
        for n in lens:
            qsl.append(qsl[-1] + n)
        seq = torch.repeat_interleave(torch.arange(len(lens), device=dev),
                                      torch.tensor(lens, device=dev))
        pos = torch.cat([torch.arange(n, device=dev) for n in lens])
        starts = torch.tensor(qsl, dtype=torch.int32, device=dev)
        meta = SimpleNamespace(query_start_loc=starts, cu_seqlens_k=starts.clone(),
                               block_table=self.block_table[:len(lens)],
                               num_seqs=len(lens), max_query_len=max(lens),
                               max_seq_len=max(lens), slot_mapping=self.slots(seq, pos))
        return meta, pos, starts[1:].long() - 1


@torch.no_grad()
def generate(model, prompts, new_tokens, graph=True, page=16, prefill_chunk=None):
    """Greedy generation for a batch of equal-length prompts [B, P]. Returns (tokens [B, N],
    prefill seconds, decode seconds). Prompts are prefilled packed, `prefill_chunk` sequences at a
    time (all by default); each decode step (one token per sequence) is captured once as a HIP
    graph and replayed (graph=True, on a GPU), as serve.py replays captured decode steps, or run
    eagerly."""
    B, P = prompts.shape
    dev = prompts.device
    batch = PagedBatch(B, P + new_tokens, page, dev)
    caches = model.new_caches(batch.num_pages, page)
    out = torch.empty(B, new_tokens, dtype=torch.long, device=dev)
    chunk = prefill_chunk or B
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for b0 in range(0, B, chunk):
        nb = min(chunk, B - b0)
        meta, pos, last = batch.prefill_meta([P] * nb)
        meta.block_table = batch.block_table[b0:b0 + nb]
        seq = torch.repeat_interleave(torch.arange(b0, b0 + nb, device=dev), P)
        meta.slot_mapping = batch.slots(seq, pos)
        logits = model(prompts[b0:b0 + nb].reshape(-1), pos, meta, caches, last)
        out[b0:b0 + nb, 0] = greedy_argmax(logits)
    torch.cuda.synchronize()
    t1 = time.perf_counter()

    # decode state, all on the device: the step reads and advances it, so it can be replayed
    tok = out[:, 0].clone()
    pos = torch.full((B,), P, dtype=torch.long, device=dev)
    col = torch.ones(1, dtype=torch.long, device=dev)
    seqs = torch.arange(B, device=dev)
    meta = SimpleNamespace(query_start_loc=torch.arange(B + 1, dtype=torch.int32, device=dev),
                           cu_seqlens_k=torch.zeros(B + 1, dtype=torch.int32, device=dev),
                           block_table=batch.block_table, num_seqs=B, max_query_len=1,
                           # the bound a captured step is valid for, as serve.py bakes
                           # max_model_len into its graph metadata (split-KV choice)
                           max_seq_len=P + new_tokens,
                           slot_mapping=torch.zeros(B, dtype=torch.long, device=dev))
    rows = torch.arange(B, device=dev)

    def step():
        meta.cu_seqlens_k[1:].copy_(torch.cumsum(pos + 1, 0))
        meta.slot_mapping.copy_(batch.slots(seqs, pos))
        nxt = greedy_argmax(model(tok, pos, meta, caches, rows))
        out.index_copy_(1, col, nxt[:, None])
        tok.copy_(nxt)
        pos.add_(1)
        col.add_(1)

    if graph and new_tokens > 1 and prompts.is_cuda:
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
        tok.copy_(out[:, 0])
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


def build_model(cfg=None, device="cuda", seed=0, router_logits="model", max_position=4096):
    cfg = cfg or Qwen3MoeConfig()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen3MoeModel(cfg, max_position, router_logits)
    finally:
        torch.set_default_dtype(torch.float32)
    model.init_random(seed)
    return model


def run_e2e(batch=64, prompt_len=512, new_tokens=256, cfg=None, seed=0, autotune=True):
    """Config 5 of the benchmark set: returns a dict of timings and throughputs. With `autotune`
    the expert plans are tuned first for batches up to the whole prefill (batch * prompt_len
    tokens), as the reference engine tunes for max_num_batched_tokens at start-up."""
    model = build_model(cfg, seed=seed)
    plans = model.autotune(batch * prompt_len) if autotune else None
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
            "first_tokens": toks[0, :8].tolist(),
            "moe_plans": None if plans is None else {b: bm for b, (bm, _) in plans.items()}}
