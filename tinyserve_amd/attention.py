"""Attention-side ops of the qwen3_moe decoder on the HIP kernels (csrc/attn.hip).

Mirrors the reference's tinykernels attention helpers, with the same argument meaning:
    qk_norm_rope     tinykernels.qk_norm_rope (tinykernels.py:220-275)
    paged_attention  tinykernels.paged_attention (tinykernels.py:891-932); `meta` carries
                     query_start_loc, cu_seqlens_k, block_table, num_seqs and max_query_len as
                     serve.AttnMetadata does (serve.py:627-637)
    greedy_argmax    the temperature-0 branch of sampling (argmax over the vocabulary)
and the paged KV cache they share (`PagedKVCache`: K pages [num_pages, page, Hkv, D] as the
reference lays them out, V pages transposed, [num_pages, Hkv, D, page], which lets the P.V
product read both matrix-core operands as they lie). All run on torch's current stream without
host synchronisation or allocation beyond their outputs, so a decode step can be captured in a
HIP graph. There is no CPU implementation.
"""
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor

from ._lib import TSM_BF16, TSM_F32, check, lib, ptr, stream_of


def _gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"tinyserve_amd attention ops run on the GPU only ({t.device})")


@dataclass
class PagedKVCache:
    """One layer's page pool. Page 0 is kept as the null page that padding tokens write to."""
    k: Tensor   # [num_pages, page, Hkv, D]
    v: Tensor   # [num_pages, Hkv, D, page]

    @staticmethod
    def allocate(num_pages: int, page: int, Hkv: int, D: int, device, dtype=torch.bfloat16):
        return PagedKVCache(torch.zeros(num_pages, page, Hkv, D, device=device, dtype=dtype),
                            torch.zeros(num_pages, Hkv, D, page, device=device, dtype=dtype))

    @property
    def page(self) -> int:
        return self.k.shape[1]


def qk_norm_rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor,
                 q_weight: Optional[Tensor] = None, k_weight: Optional[Tensor] = None,
                 eps: float = 1e-6, v: Optional[Tensor] = None,
                 cache: Optional[PagedKVCache] = None,
                 slot_mapping: Optional[Tensor] = None):
    """In place on q [T, H, D] and k [T, Hkv, D]: per-head RMSNorm (if weights), rotate-half RoPE
    with cos/sin [T, D/2] fp32; with a cache, also writes k and v at slot_mapping [T] (int64)."""
    _gpu(q, k, cos, sin, v, slot_mapping)
    T, H, D = q.shape
    Hkv = k.shape[1]
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise TypeError("qk_norm_rope runs in bf16")
    if q.stride(-1) != 1 or k.stride(-1) != 1:
        raise ValueError("q and k heads must be contiguous in the last dimension")
    cos, sin = cos.float(), sin.float()
    if cos.stride(-1) != 1 or sin.stride(-1) != 1 or cos.stride(0) != sin.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    if (q_weight is None) != (k_weight is None):
        raise ValueError("q and k norm weights come together")
    kc = vc = None
    page = num_pages = 0
    if cache is not None:
        if v is None or slot_mapping is None:
            raise ValueError("a cache write needs v and slot_mapping")
        if v.stride(-1) != 1:
            raise ValueError("v heads must be contiguous in the last dimension")
        kc, vc, page, num_pages = cache.k, cache.v, cache.page, cache.k.shape[0]
        slot_mapping = slot_mapping.to(torch.int64).contiguous()
    check(lib.tsm_qk_norm_rope(
        ptr(q), T, H, q.stride(0), q.stride(1), ptr(k), Hkv, k.stride(0), k.stride(1),
        ptr(v), v.stride(0) if v is not None else 0, v.stride(1) if v is not None else 0, D,
        ptr(cos), ptr(sin), cos.stride(0), ptr(q_weight), ptr(k_weight), float(eps), ptr(kc),
        ptr(vc), num_pages, page, ptr(slot_mapping), stream_of(q)), "qk_norm_rope")
    return q, k


def paged_attention(q: Tensor, cache: PagedKVCache, meta, scale: float) -> Tensor:
    """Causal attention of the packed queries q [T, H, D] over each request's paged context.
    meta: query_start_loc [B+1] i32, cu_seqlens_k [B+1] i32, block_table [B, max_pages] i32,
    num_seqs, max_query_len (as serve.AttnMetadata)."""
    _gpu(q, cache.k, cache.v)
    T, H, D = q.shape
    Hkv = cache.k.shape[2]
    if q.stride(-1) != 1:
        q = q.contiguous()
    out = torch.empty(T, H, D, dtype=q.dtype, device=q.device)
    qsl = meta.query_start_loc.to(torch.int32).contiguous()
    cuk = meta.cu_seqlens_k.to(torch.int32).contiguous()
    bt = meta.block_table
    if bt.dtype != torch.int32 or bt.stride(-1) != 1:
        bt = bt.to(torch.int32).contiguous()
    check(lib.tsm_paged_attention(
        ptr(q), T, H, q.stride(0), q.stride(1), ptr(cache.k), ptr(cache.v), cache.k.shape[0],
        cache.page, Hkv, D,
        ptr(qsl), ptr(cuk), ptr(bt), bt.stride(0), int(meta.num_seqs), int(meta.max_query_len),
        float(scale), ptr(out), out.stride(0), out.stride(1), stream_of(q)), "paged_attention")
    return out


def greedy_argmax(logits: Tensor) -> Tensor:
    """Index of the largest logit per row (lowest index among ties), int64 [rows]."""
    _gpu(logits)
    if logits.dtype not in (torch.float32, torch.bfloat16):
        logits = logits.float()
    x = logits.reshape(-1, logits.shape[-1])
    if x.stride(-1) != 1:
        x = x.contiguous()
    out = torch.empty(x.shape[0], dtype=torch.int64, device=x.device)
    check(lib.tsm_greedy_argmax(ptr(x), TSM_F32 if x.dtype == torch.float32 else TSM_BF16,
                                x.shape[0], x.stride(0), x.shape[1], ptr(out), stream_of(x)),
          "greedy_argmax")
    return out.view(logits.shape[:-1])
