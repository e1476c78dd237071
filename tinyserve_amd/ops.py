"""PyTorch custom ops (namespace `tinyserve_amd`) over the C ABI of libtinyserve_moe.so.

Every op validates shapes/dtypes/devices here, allocates its outputs and workspace with torch's
caching allocator, and launches on torch's current stream; nothing synchronises the host, so the
ops can be captured into a HIP graph (torch.cuda.graph). There is no CPU implementation: a CPU
tensor raises.
"""
from typing import Optional, Tuple

import torch
from torch import Tensor

import ctypes
import weakref

from ._lib import TSM_BF16, TSM_F32, check, lib, ptr, stream_of


def _on_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"tinyserve_amd ops run on the GPU only (got a tensor on {t.device}); "
                "there is no CPU implementation")


def _contig(t: Tensor) -> Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _map_arg(expert_map: Optional[Tensor], device) -> Optional[Tensor]:
    if expert_map is None:
        return None
    return _contig(expert_map.to(device=device, dtype=torch.int64))


# ---------------------------------------------------------------- routing
@torch.library.custom_op("tinyserve_amd::moe_route", mutates_args=())
def moe_route(logits: Tensor, top_k: int, renormalize: bool,
              expert_map: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """logits [T, E] -> (topk_weights fp32 [T, k], topk_ids int32 [T, k])."""
    _on_gpu(logits, expert_map)
    if logits.dim() != 2:
        raise ValueError(f"logits must be [T, E], got {tuple(logits.shape)}")
    if logits.dtype not in (torch.float32, torch.bfloat16):
        logits = logits.float()
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    T, E = logits.shape
    w = torch.empty(T, top_k, dtype=torch.float32, device=logits.device)
    ids = torch.empty(T, top_k, dtype=torch.int32, device=logits.device)
    m = _map_arg(expert_map, logits.device)
    dt = TSM_F32 if logits.dtype == torch.float32 else TSM_BF16
    check(lib.tsm_moe_route(ptr(logits), dt, T, E, logits.stride(0), top_k, int(renormalize),
                            ptr(m), ptr(w), ptr(ids), stream_of(logits)), "moe_route")
    return w, ids


@moe_route.register_fake
def _(logits, top_k, renormalize, expert_map=None):
    T = logits.shape[0]
    return (logits.new_empty(T, top_k, dtype=torch.float32),
            logits.new_empty(T, top_k, dtype=torch.int32))


@torch.library.custom_op("tinyserve_amd::moe_router", mutates_args=())
def moe_router(x: Tensor, gate_w: Tensor, top_k: int, renormalize: bool,
               expert_map: Optional[Tensor] = None, bias: Optional[Tensor] = None,
               logits_bf16: bool = False) -> Tuple[Tensor, Tensor, Tensor]:
    """Gate GEMM + routing: -> (topk_weights, topk_ids, fp32 logits [T, E]). One launch; two at
    decode sizes (T <= 256: the gate GEMM spread over expert slices, then the selection)."""
    _on_gpu(x, gate_w, expert_map, bias)
    if x.dtype != gate_w.dtype or x.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"router needs x and gate weight both bf16 or both fp32, got "
                        f"{x.dtype}/{gate_w.dtype}")
    x, gate_w = _contig(x), _contig(gate_w)
    T, H = x.shape
    E = gate_w.shape[0]
    if gate_w.shape[1] != H:
        raise ValueError(f"gate weight {tuple(gate_w.shape)} does not match x {tuple(x.shape)}")
    if H % 8:
        # the kernels read rows in 8-element chunks: zero columns add exact zeros to every
        # partial sum, so the logits keep their bits
        H = (H + 7) // 8 * 8
        x, gate_w = _pad_cols(x, H), _pad_cols(gate_w, H)
    w = torch.empty(T, top_k, dtype=torch.float32, device=x.device)
    ids = torch.empty(T, top_k, dtype=torch.int32, device=x.device)
    logits = torch.empty(T, E, dtype=torch.float32, device=x.device)
    m = _map_arg(expert_map, x.device)
    b = None if bias is None else _contig(bias.to(device=x.device, dtype=torch.float32))
    dt = TSM_BF16 if x.dtype == torch.bfloat16 else TSM_F32
    check(lib.tsm_moe_router(ptr(x), ptr(gate_w), dt, T, H, E, top_k, int(renormalize), ptr(m),
                             ptr(b), int(logits_bf16), ptr(logits), ptr(w), ptr(ids),
                             stream_of(x)), "moe_router")
    return w, ids, logits


@moe_router.register_fake
def _(x, gate_w, top_k, renormalize, expert_map=None, bias=None, logits_bf16=False):
    T, E = x.shape[0], gate_w.shape[0]
    return (x.new_empty(T, top_k, dtype=torch.float32), x.new_empty(T, top_k, dtype=torch.int32),
            x.new_empty(T, E, dtype=torch.float32))


# ---------------------------------------------------------------- permutation
@torch.library.custom_op("tinyserve_amd::moe_align_block_size", mutates_args=())
def moe_align_block_size(topk_ids: Tensor, block_m: int,
                         num_experts: int) -> Tuple[Tensor, Tensor, Tensor]:
    """-> (sorted_ids int32 [max_padded], expert_ids int32 [max_padded/block_m], total int32 [1])"""
    _on_gpu(topk_ids)
    flat = _contig(topk_ids.reshape(-1).to(torch.int32))
    numel = flat.numel()
    mp = int(lib.tsm_moe_max_padded(numel, num_experts, block_m))
    if mp < 0:
        raise ValueError("invalid num_experts / block_m")
    dev = topk_ids.device
    sorted_ids = torch.empty(mp, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(mp // block_m, dtype=torch.int32, device=dev)
    total = torch.empty(1, dtype=torch.int32, device=dev)
    nws = int(lib.tsm_moe_align_workspace_size(numel, num_experts, block_m))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=dev)
    check(lib.tsm_moe_align(ptr(flat), numel, num_experts, block_m, ptr(sorted_ids),
                            ptr(expert_ids), ptr(total), ptr(ws), nws, stream_of(flat)),
          "moe_align_block_size")
    return sorted_ids, expert_ids, total


@moe_align_block_size.register_fake
def _(topk_ids, block_m, num_experts):
    numel = topk_ids.numel()
    nb = num_experts + 1
    mp = -(-(numel + nb * (block_m - 1)) // block_m) * block_m
    return (topk_ids.new_empty(mp, dtype=torch.int32),
            topk_ids.new_empty(mp // block_m, dtype=torch.int32),
            topk_ids.new_empty(1, dtype=torch.int32))


# ---------------------------------------------------------------- activation
@torch.library.custom_op("tinyserve_amd::silu_and_mul", mutates_args=())
def silu_and_mul(gate: Tensor, up: Tensor) -> Tensor:
    """bf16(bf16(silu(gate)) * up) over the last dimension (strided rows allowed)."""
    _on_gpu(gate, up)
    if gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise TypeError("silu_and_mul supports bf16 tensors")
    if gate.shape != up.shape:
        raise ValueError("gate and up shapes differ")
    shape = gate.shape
    N = shape[-1]
    a, b = gate.reshape(-1, N), up.reshape(-1, N)
    if a.stride(-1) != 1:
        a = a.contiguous()
    if b.stride(-1) != 1:
        b = b.contiguous()
    out = torch.empty(a.shape, dtype=gate.dtype, device=gate.device)
    check(lib.tsm_silu_and_mul(ptr(a), a.stride(0), ptr(b), b.stride(0), ptr(out), out.stride(0),
                               a.shape[0], N, stream_of(a)), "silu_and_mul")
    return out.view(shape)


@silu_and_mul.register_fake
def _(gate, up):
    return torch.empty_like(gate)


# ---------------------------------------------------------------- experts
def padded_shape(H: int, I: int) -> Tuple[int, int]:
    """(H_pad, I_pad): the sizes the expert kernels run at (equal to (H, I) when the kernels
    take those sizes; else rounded up, with the margin of the packed weights zero)."""
    hp, ip = ctypes.c_int(0), ctypes.c_int(0)
    check(lib.tsm_moe_padded_shape(H, I, ctypes.byref(hp), ctypes.byref(ip)), "padded_shape")
    return hp.value, ip.value


def _needs_padding(H: int, I: int) -> bool:
    return padded_shape(H, I) != (H, I)


def _check_weights(x, w13, w2):
    if x.dtype != torch.bfloat16 or w13.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16:
        raise TypeError(f"fused_moe runs in bf16, or fp32 in the reference layout (got x "
                        f"{x.dtype}, w13 {w13.dtype}, w2 {w2.dtype})")
    T, H = x.shape
    E, two_i, H1 = w13.shape
    I = two_i // 2
    if H1 != H or tuple(w2.shape) != (E, H, I) or two_i != 2 * I:
        raise ValueError(f"weight shapes w13 {tuple(w13.shape)} / w2 {tuple(w2.shape)} do not "
                         f"match x {tuple(x.shape)}")
    return T, H, E, I


def _check_packed(x, w13p, w2p):
    """Packed weights may carry the padded sizes of padded_shape(H, I): w13p [E, 2 I_pad, H_pad],
    w2p [E, H_pad, I_pad]. Returns (T, H, H_pad, E, I_pad)."""
    if x.dtype != torch.bfloat16 or w13p.dtype != torch.bfloat16 or w2p.dtype != torch.bfloat16:
        raise TypeError(f"fused_moe runs in bf16 (got x {x.dtype}, w13 {w13p.dtype}, "
                        f"w2 {w2p.dtype})")
    T, H = x.shape
    E, two_i, Hp = w13p.shape
    Ip = two_i // 2
    if tuple(w2p.shape) != (E, Hp, Ip) or two_i != 2 * Ip:
        raise ValueError(f"packed weight shapes w13 {tuple(w13p.shape)} / w2 {tuple(w2p.shape)} "
                         f"are inconsistent")
    if Hp != H and padded_shape(H, Ip)[0] != Hp:
        raise ValueError(f"packed weights have H={Hp}, which is neither x's H={H} nor its "
                         f"padded size {padded_shape(H, Ip)[0]}")
    return T, H, Hp, E, Ip


def _pad_cols(x, n):
    return x if x.shape[1] == n else torch.nn.functional.pad(x, (0, n - x.shape[1]))


def _fused_moe_f32(x, w13, w2, topk_weights, topk_ids, sum_topk):
    """fp32 layer: every intermediate in fp32 (the reference keeps them in x.dtype)."""
    T, H = x.shape
    E, two_i, H1 = w13.shape
    I = two_i // 2
    if H1 != H or tuple(w2.shape) != (E, H, I) or two_i != 2 * I:
        raise ValueError(f"weight shapes w13 {tuple(w13.shape)} / w2 {tuple(w2.shape)} do not "
                         f"match x {tuple(x.shape)}")
    k = topk_ids.shape[1]
    tw = _contig(topk_weights.to(torch.float32))
    ti = _contig(topk_ids.to(torch.int32))
    out = torch.empty((T, H) if sum_topk else (T * k, H), dtype=x.dtype, device=x.device)
    nws = int(lib.tsm_fused_moe_f32_workspace_size(T, H, I, E, k))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=x.device)
    check(lib.tsm_fused_moe_f32(ptr(x), ptr(w13), ptr(w2), ptr(tw), ptr(ti), T, H, I, E, k,
                                int(sum_topk), ptr(out), ptr(ws), nws, stream_of(x)),
          "fused_moe (fp32)")
    return out


def _fused_moe_impl(x, w13, w2, topk_weights, topk_ids, sum_topk, packed):
    _on_gpu(x, w13, w2, topk_weights, topk_ids)
    x, w13, w2 = _contig(x), _contig(w13), _contig(w2)
    if not packed and x.dtype == torch.float32 and w13.dtype == torch.float32 \
            and w2.dtype == torch.float32:
        return _fused_moe_f32(x, w13, w2, topk_weights, topk_ids, sum_topk)
    if not packed:
        T, H, E, I = _check_weights(x, w13, w2)
        if _needs_padding(H, I):
            # a shape the kernels do not take as it is: run on a zero-padded packed copy
            w13, w2 = _padded_pack_cached(w13, w2)
            packed = True
    if packed:
        T, H, Hp, E, Ip = _check_packed(x, w13, w2)
    else:
        Hp, Ip = H, I
    k = topk_ids.shape[1]
    tw = _contig(topk_weights.to(torch.float32))
    ti = _contig(topk_ids.to(torch.int32))
    xp = _pad_cols(x, Hp)
    out = torch.empty((T, Hp) if sum_topk else (T * k, Hp), dtype=x.dtype, device=x.device)
    nws = int(lib.tsm_fused_moe_workspace_size(T, Hp, Ip, E, k))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=x.device)
    fn = lib.tsm_fused_moe_packed if packed else lib.tsm_fused_moe
    check(fn(ptr(xp), ptr(w13), ptr(w2), ptr(tw), ptr(ti), T, Hp, Ip, E, k, int(sum_topk),
             ptr(out), ptr(ws), nws, stream_of(x)), "fused_moe")
    return out if Hp == H else out[:, :H].contiguous()


# Zero-padded packed copies made for reference-layout weights whose shape the kernels do not take
# as it is, one per weight tensor (dropped with it), rebuilt when either tensor's storage or
# version counter moves. Keyed by id() with a weak reference checked by identity: a
# WeakKeyDictionary would compare two tensors with == (elementwise) on a repeated lookup.
_padded_cache: dict = {}


def _padded_pack_cached(w13, w2):
    key = (w13.data_ptr(), w2.data_ptr(), w13._version, w2._version)
    hit = _padded_cache.get(id(w13))
    if hit is not None and hit[0]() is w13 and hit[1] == key:
        return hit[2]
    with torch.no_grad():
        p = pack_moe_weights(w13, w2)
    i = id(w13)

    def drop(r, i=i):
        if _padded_cache.get(i, (None,))[0] is r:
            del _padded_cache[i]

    _padded_cache[i] = (weakref.ref(w13, drop), key, p)
    return p


@torch.library.custom_op("tinyserve_amd::fused_moe", mutates_args=())
def fused_moe(x: Tensor, w13: Tensor, w2: Tensor, topk_weights: Tensor, topk_ids: Tensor,
              sum_topk: bool = True) -> Tensor:
    """sum_k weight_k * expert_k(x) -> [T, H] (or the per-slot rows [T*k, H])."""
    return _fused_moe_impl(x, w13, w2, topk_weights, topk_ids, sum_topk, False)


@fused_moe.register_fake
def _(x, w13, w2, topk_weights, topk_ids, sum_topk=True):
    T, H = x.shape
    k = topk_ids.shape[1]
    return x.new_empty((T, H) if sum_topk else (T * k, H))


@torch.library.custom_op("tinyserve_amd::fused_moe_packed", mutates_args=())
def fused_moe_packed(x: Tensor, w13_packed: Tensor, w2_packed: Tensor, topk_weights: Tensor,
                     topk_ids: Tensor, sum_topk: bool = True) -> Tensor:
    """fused_moe on weights reordered by pack_moe_weights (same shapes as w13 / w2)."""
    return _fused_moe_impl(x, w13_packed, w2_packed, topk_weights, topk_ids, sum_topk, True)


@fused_moe_packed.register_fake
def _(x, w13_packed, w2_packed, topk_weights, topk_ids, sum_topk=True):
    T, H = x.shape
    k = topk_ids.shape[1]
    return x.new_empty((T, H) if sum_topk else (T * k, H))


@torch.library.custom_op("tinyserve_amd::pack_moe_weights", mutates_args=())
def pack_moe_weights(w13: Tensor, w2: Tensor) -> Tuple[Tensor, Tensor]:
    """MFMA-tiled copies of w13 [E, 2I, H] and w2 [E, H, I]; one-time, at weight-load time. Same
    shapes when the kernels take (H, I) as they are; otherwise [E, 2 I_pad, H_pad] and
    [E, H_pad, I_pad] (padded_shape) with a zero margin. Their contents are only meaningful to
    the *_packed ops."""
    _on_gpu(w13, w2)
    if w13.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16:
        raise TypeError("packing supports bf16 weights")
    w13, w2 = _contig(w13), _contig(w2)
    E, two_i, H = w13.shape
    I = two_i // 2
    if tuple(w2.shape) != (E, H, I) or two_i != 2 * I:
        raise ValueError(f"w2 {tuple(w2.shape)} does not match w13 {tuple(w13.shape)}")
    Hp, Ip = padded_shape(H, I)
    p13 = torch.empty(E, 2 * Ip, Hp, dtype=w13.dtype, device=w13.device)
    p2 = torch.empty(E, Hp, Ip, dtype=w2.dtype, device=w2.device)
    s = stream_of(w13)
    check(lib.tsm_moe_pack_weights_padded(ptr(w13), E, two_i, H, 2 * Ip, Hp, 1, ptr(p13), s),
          "pack w13")
    check(lib.tsm_moe_pack_weights_padded(ptr(w2), E, H, I, Hp, Ip, 0, ptr(p2), s), "pack w2")
    return p13, p2


@pack_moe_weights.register_fake
def _(w13, w2):
    E, two_i, H = w13.shape
    Hp, Ip = padded_shape(H, two_i // 2)
    return w13.new_empty(E, 2 * Ip, Hp), w2.new_empty(E, Hp, Ip)


def _moe_forward_impl(x, gate_w, w13, w2, top_k, renormalize, expert_map, bias, logits_bf16,
                      sum_topk, packed):
    _on_gpu(x, gate_w, w13, w2, expert_map, bias)
    x, gate_w, w13, w2 = _contig(x), _contig(gate_w), _contig(w13), _contig(w2)
    if not packed and x.dtype == torch.float32:
        # fp32 layer: the fused router (fp32 inputs) then the fp32 experts
        w, ids, _ = moe_router(x, gate_w, top_k, renormalize, expert_map, bias, logits_bf16)
        return _fused_moe_impl(x, w13, w2, w, ids, sum_topk, False)
    if packed:
        T, H, Hp, E, Ip = _check_packed(x, w13, w2)
        ragged = Hp != H
    else:
        T, H, E, I = _check_weights(x, w13, w2)
        ragged = _needs_padding(H, I)
    if gate_w.dtype != torch.bfloat16 or tuple(gate_w.shape) != (E, H):
        raise ValueError(f"gate weight must be bf16 [E, H] = [{E}, {H}]")
    if ragged:
        # router on the true hidden size, experts on the padded one
        w, ids, _ = moe_router(x, gate_w, top_k, renormalize, expert_map, bias, logits_bf16)
        return _fused_moe_impl(x, w13, w2, w, ids, sum_topk, packed)
    if not packed:
        Ip = I
    m = _map_arg(expert_map, x.device)
    b = None if bias is None else _contig(bias.to(device=x.device, dtype=torch.float32))
    out = torch.empty((T, H) if sum_topk else (T * top_k, H), dtype=x.dtype, device=x.device)
    nws = int(lib.tsm_moe_forward_workspace_size(T, H, Ip, E, top_k))
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device=x.device)
    fn = lib.tsm_moe_forward_packed if packed else lib.tsm_moe_forward
    check(fn(ptr(x), ptr(gate_w), ptr(w13), ptr(w2), ptr(m), ptr(b), T, H, Ip, E, top_k,
             int(renormalize), int(logits_bf16), int(sum_topk), ptr(out), None, None, ptr(ws),
             nws, stream_of(x)), "moe_forward")
    return out


@torch.library.custom_op("tinyserve_amd::moe_forward", mutates_args=())
def moe_forward(x: Tensor, gate_w: Tensor, w13: Tensor, w2: Tensor, top_k: int,
                renormalize: bool, expert_map: Optional[Tensor] = None,
                bias: Optional[Tensor] = None, logits_bf16: bool = False,
                sum_topk: bool = True) -> Tensor:
    """Whole MoE block: fused router (gate GEMM + softmax/top-k) then the experts."""
    return _moe_forward_impl(x, gate_w, w13, w2, top_k, renormalize, expert_map, bias,
                             logits_bf16, sum_topk, False)


@moe_forward.register_fake
def _(x, gate_w, w13, w2, top_k, renormalize, expert_map=None, bias=None, logits_bf16=False,
      sum_topk=True):
    T, H = x.shape
    return x.new_empty((T, H) if sum_topk else (T * top_k, H))


@torch.library.custom_op("tinyserve_amd::moe_forward_packed", mutates_args=())
def moe_forward_packed(x: Tensor, gate_w: Tensor, w13_packed: Tensor, w2_packed: Tensor,
                       top_k: int, renormalize: bool, expert_map: Optional[Tensor] = None,
                       bias: Optional[Tensor] = None, logits_bf16: bool = False,
                       sum_topk: bool = True) -> Tensor:
    """moe_forward on weights reordered by pack_moe_weights."""
    return _moe_forward_impl(x, gate_w, w13_packed, w2_packed, top_k, renormalize, expert_map,
                             bias, logits_bf16, sum_topk, True)


@moe_forward_packed.register_fake
def _(x, gate_w, w13_packed, w2_packed, top_k, renormalize, expert_map=None, bias=None,
      logits_bf16=False, sum_topk=True):
    T, H = x.shape
    return x.new_empty((T, H) if sum_topk else (T * top_k, H))


# ---------------------------------------------------------------- residual-add RMSNorm
def _norm_impl(x, top_k, residual, residual_in, weight, eps):
    _on_gpu(x, residual, weight)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError(f"add_rmsnorm runs in bf16 (got x {x.dtype}, weight {weight.dtype})")
    H = x.shape[-1]
    x2 = _contig(x.reshape(-1, H))
    if x2.shape[0] % top_k:
        raise ValueError(f"{x2.shape[0]} rows are not a whole number of tokens of {top_k} slots")
    T = x2.shape[0] // top_k
    if tuple(weight.shape) != (H,):
        raise ValueError(f"weight {tuple(weight.shape)} does not match H={H}")
    if residual is not None and (residual.dtype != torch.bfloat16 or residual.numel() != T * H
                                 or not residual.is_contiguous()):
        raise ValueError("residual must be a contiguous bf16 tensor of T*H elements")
    out = torch.empty(T, H, dtype=x.dtype, device=x.device)
    check(lib.tsm_add_rmsnorm(ptr(x2), T, H, top_k, ptr(residual), int(residual_in),
                              ptr(_contig(weight)), float(eps), ptr(out), stream_of(x2)),
          "add_rmsnorm")
    return out


@torch.library.custom_op("tinyserve_amd::add_rmsnorm", mutates_args=("residual",))
def _add_rmsnorm(x: Tensor, top_k: int, residual: Optional[Tensor], residual_in: bool,
                 weight: Tensor, eps: float) -> Tensor:
    return _norm_impl(x, top_k, residual, residual_in, weight, eps)


@_add_rmsnorm.register_fake
def _(x, top_k, residual, residual_in, weight, eps):
    H = x.shape[-1]
    return x.new_empty(x.numel() // H // top_k, H)


def rmsnorm(x: Tensor, weight: Tensor, eps: float, residual: Optional[Tensor] = None) -> Tensor:
    """tinykernels.rmsnorm (tinykernels.py:63-105): out = rmsnorm(x) * weight, or with a residual
    `residual += x` (rounded to bf16) then out = rmsnorm(residual) * weight, in one launch."""
    return _add_rmsnorm(x, 1, residual, residual is not None, weight, eps).view(x.shape)


def moe_combine_add_rmsnorm(rows: Tensor, top_k: int, residual: Tensor, weight: Tensor,
                            eps: float, residual_in: bool = True) -> Tensor:
    """The MoE block's k-sum fused into the next residual-add RMSNorm: rows [T*k, H] (fused_moe
    with sum_topk=False) -> residual = bf16(bf16(sum_k rows) + residual) (residual_in; else
    residual = bf16(sum_k rows)), returns rmsnorm(residual) * weight [T, H]."""
    if residual is None:
        raise ValueError("moe_combine_add_rmsnorm needs a residual buffer")
    return _add_rmsnorm(rows, top_k, residual, residual_in, weight, eps)
