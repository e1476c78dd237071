"""Attention-side ops of the qwen3_moe decoder on the HIP kernels (csrc/attn.hip).

Mirrors the reference's tinykernels attention helpers, with the same argument meaning:
    qk_norm_rope     tinykernels.qk_norm_rope (tinykernels.py:220-275)
    paged_attention  tinykernels.paged_attention (tinykernels.py:891-932), split-KV decode
                     included; `meta` carries query_start_loc, cu_seqlens_k, block_table,
                     num_seqs, max_query_len and max_seq_len as serve.AttnMetadata does
                     (serve.py:627-637)
    greedy_argmax    the temperature-0 branch of sampling (argmax over the vocabulary)
with the reference's signatures, on the page pools the reference passes (k_cache, v_cache), with
one layout difference: K pages are [num_pages, page, Hkv, D] as the reference lays them out, V
pages are transposed, [num_pages, Hkv, D, page], which lets the P.V product read both
matrix-core operands as they lie (`PagedKVCache.allocate` makes such a pair). All run on torch's current stream without
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


def _check_caches(k_cache: Tensor, v_cache: Tensor, Hkv: int, D: int):
    """K pages [num_pages, page, Hkv, D]; V pages transposed, [num_pages, Hkv, D, page]."""
    n, page = k_cache.shape[0], k_cache.shape[1]
    if tuple(k_cache.shape) != (n, page, Hkv, D) or tuple(v_cache.shape) != (n, Hkv, D, page):
        raise ValueError(f"caches must be K [num_pages, page, Hkv, D] and V [num_pages, Hkv, D, "
                         f"page] (V transposed); got {tuple(k_cache.shape)} and "
                         f"{tuple(v_cache.shape)} for Hkv={Hkv}, D={D}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("the page pools must be contiguous")
    return n, page


def qk_norm_rope(q: Tensor, k: Tensor, cos: Tensor, sin: Tensor,
                 q_weight: Optional[Tensor] = None, k_weight: Optional[Tensor] = None,
                 eps: float = 1e-6, v: Optional[Tensor] = None,
                 k_cache: Optional[Tensor] = None, v_cache: Optional[Tensor] = None,
                 slot_mapping: Optional[Tensor] = None):
    """In place on q [T, H, D] and k [T, Hkv, D]: per-head RMSNorm (if weights), rotate-half RoPE
    with cos/sin [T, D/2] fp32; with slot_mapping [T] (int64), also writes k and v into the page
    pools k_cache / v_cache (V pages transposed, see PagedKVCache)."""
    _gpu(q, k, cos, sin, v, k_cache, v_cache, slot_mapping)
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
    if slot_mapping is not None:
        if v is None or k_cache is None or v_cache is None:
            raise ValueError("a cache write needs v, k_cache and v_cache")
        if v.stride(-1) != 1:
            raise ValueError("v heads must be contiguous in the last dimension")
        num_pages, page = _check_caches(k_cache, v_cache, Hkv, D)
        kc, vc = k_cache, v_cache
        slot_mapping = slot_mapping.to(torch.int64).contiguous()
    check(lib.tsm_qk_norm_rope(
        ptr(q), T, H, q.stride(0), q.stride(1), ptr(k), Hkv, k.stride(0), k.stride(1),
        ptr(v), v.stride(0) if v is not None else 0, v.stride(1) if v is not None else 0, D,
        ptr(cos), ptr(sin), cos.stride(0), ptr(q_weight), ptr(k_weight), float(eps), ptr(kc),
        ptr(vc), num_pages, page, ptr(slot_mapping), stream_of(q)), "qk_norm_rope")
    return q, k


_cu_counts = {}


def choose_num_splits(programs: int, max_seq_len: Optional[int], device) -> int:
    """Split-KV factor for a decode launch of `programs` = B * Hkv workgroups: enough splits for
    about two workgroups per CU, none shorter than 256 keys, at most 16, a power of two (the
    reference's rule, tinykernels.py:865-889). Without a known max_seq_len: no split."""
    if not max_seq_len or programs <= 0:
        return 1
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _cu_counts:
        _cu_counts[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    want = -(-2 * _cu_counts[idx] // programs)
    s = min(want, max(1, int(max_seq_len) // 256), 16)
    return 1 if s <= 1 else 1 << (s - 1).bit_length()


def paged_attention(q: Tensor, k_cache: Tensor, v_cache: Tensor, meta, scale: float,
                    num_splits: Optional[int] = None) -> Tensor:
    """Causal attention of the packed queries q [T, H, D] over each request's paged context.
    meta: query_start_loc [B+1] i32, cu_seqlens_k [B+1] i32, block_table [B, max_pages] i32,
    num_seqs, max_query_len, and (for the split-KV choice) max_seq_len, as serve.AttnMetadata.
    num_splits: split-KV factor of the one-token requests (None: chosen from B * Hkv and
    max_seq_len like the reference; 1: no split)."""
    _gpu(q, k_cache, v_cache)
    T, H, D = q.shape
    Hkv = k_cache.shape[2]
    num_pages, page = _check_caches(k_cache, v_cache, Hkv, D)
    if q.stride(-1) != 1:
        q = q.contiguous()
    B = int(meta.num_seqs)
    if num_splits is None:
        num_splits = choose_num_splits(B * Hkv, getattr(meta, "max_seq_len", None), q.device)
    out = torch.empty(T, H, D, dtype=q.dtype, device=q.device)
    qsl = meta.query_start_loc.to(torch.int32).contiguous()
    cuk = meta.cu_seqlens_k.to(torch.int32).contiguous()
    bt = meta.block_table
    if bt.dtype != torch.int32 or bt.stride(-1) != 1:
        bt = bt.to(torch.int32).contiguous()
    nws = int(lib.tsm_paged_attention_workspace_size(B, H, D, int(num_splits)))
    ws = torch.empty(nws, dtype=torch.uint8, device=q.device) if nws else None
    check(lib.tsm_paged_attention(
        ptr(q), T, H, q.stride(0), q.stride(1), ptr(k_cache), ptr(v_cache), num_pages, page, Hkv,
        D, ptr(qsl), ptr(cuk), ptr(bt), bt.stride(0), B, int(meta.max_query_len), float(scale),
        int(num_splits), ptr(ws), nws, ptr(out), out.stride(0), out.stride(1), stream_of(q)),
        "paged_attention")
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
