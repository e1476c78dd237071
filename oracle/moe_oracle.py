"""Torch-CPU / numpy restatement of the reference MoE path (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the checker; the product package never does.

Functions and the reference code they restate:
- moe_reference            serve.py:933-996   per-expert loop: rows routed to expert e go through
                                              x @ w13[e].T (bf16 result), silu(gate) * up, then
                                              (h @ w2[e].T).float() * weight, index-added into an fp32
                                              [T, H] accumulator in expert order; cast to x.dtype.
- route_torch              serve.py:1089-1096 fp32 softmax of the logits, top-k (ties: lowest index,
                                              which this build defines; torch.topk leaves it open),
                                              optional renormalisation, expert_map lookup.
- moe_align_block_size_np  tinykernels.py:1070-1190 (the torch moe_align_block_size).
- sparse_moe_reference     serve.py:1076-1099 at TP=1 with TRITON_KERNELS off: gate Linear, route,
                                              moe_reference.
- silu_and_mul_reference   tinykernels.py:293-297 / serve.py's F.silu(gate) * up in bf16: silu of
                                              the fp32 gate rounded to bf16, times up, rounded.
- add_rmsnorm_reference    serve.py:799-809 (RMSNorm, fp32) and 1185-1193 (add_rmsnorm: residual
                                              = residual + x in bf16, then the norm), with x the
                                              k-sum of the per-slot rows as tinykernels.py:1796
                                              forms it (fp32 sum in slot order, rounded once).
- per_token_fp64           textbook formula sum_k w_k * W2_e (silu(W1_e x) * W3_e x) in float64,
                           used only to pin moe_reference itself.
"""
import numpy as np
import torch
import torch.nn.functional as F


def moe_reference(x, w13, w2, topk_weights, topk_ids):
    """x [T,H], w13 [E,2I,H] (gate rows then up rows), w2 [E,H,I], topk_* [T,k]."""
    T, H = x.shape
    I = w2.shape[-1]
    acc = torch.zeros(T, H, dtype=torch.float32, device=x.device)
    for e in range(w13.shape[0]):
        hit = topk_ids == e
        if not bool(hit.any()):
            continue
        tok, slot = hit.nonzero(as_tuple=True)
        gu = x[tok] @ w13[e].t()                     # [n, 2I] in x.dtype
        act = F.silu(gu[:, :I]) * gu[:, I:]          # SwiGLU, in x.dtype
        y = (act @ w2[e].t()).float()                # [n, H]
        acc.index_add_(0, tok, y * topk_weights[tok, slot].unsqueeze(1).float())
    return acc.to(x.dtype)


def moe_rows_reference(x, w13, w2, topk_weights, topk_ids):
    """Per-(token, slot) rows: row t*k+s = bf16(expert(x_t) * w) as the fused kernel's sum_topk=False
    output (tinykernels.py:1791-1796); zeros for ids outside [0, E)."""
    T, H = x.shape
    k = topk_ids.shape[1]
    I = w2.shape[-1]
    rows = torch.zeros(T * k, H, dtype=x.dtype)
    for e in range(w13.shape[0]):
        hit = topk_ids == e
        if not bool(hit.any()):
            continue
        tok, slot = hit.nonzero(as_tuple=True)
        gu = x[tok] @ w13[e].t()
        act = F.silu(gu[:, :I]) * gu[:, I:]
        y = (act @ w2[e].t()).float() * topk_weights[tok, slot].unsqueeze(1).float()
        rows[tok * k + slot] = y.to(x.dtype)
    return rows


def route_torch(logits, top_k, renorm, expert_map=None):
    """serve.py:1089-1096 with an explicit lowest-index tie-break (stable descending sort)."""
    probs = logits.float().softmax(-1)
    order = torch.sort(probs, dim=-1, descending=True, stable=True).indices[:, :top_k]
    w = torch.gather(probs, 1, order)
    if renorm:
        w = w / w.sum(-1, keepdim=True)
    ids = order if expert_map is None else expert_map[order]
    return w, ids


def sparse_moe_reference(x, gate_w, w13, w2, top_k, renorm, expert_map=None):
    logits = x @ gate_w.t()
    w, ids = route_torch(logits, top_k, renorm, expert_map)
    return moe_reference(x, w13, w2, w, ids)


def moe_align_block_size_np(topk_ids, block_m, num_experts):
    """numpy restatement of moe_align_block_size (tinykernels.py:1070-1190)."""
    flat = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    flat = np.where((flat < 0) | (flat >= num_experts), num_experts, flat)
    nb = num_experts + 1
    numel = flat.size
    max_padded = -(-(numel + nb * (block_m - 1)) // block_m) * block_m
    counts = np.bincount(flat, minlength=nb)
    padded = -(-counts // block_m) * block_m
    padded_end = np.cumsum(padded)
    padded_start = padded_end - padded
    count_start = np.cumsum(counts) - counts
    order = np.argsort(flat, kind="stable")
    experts_sorted = flat[order]
    rank = np.arange(numel) - count_start[experts_sorted]
    dest = padded_start[experts_sorted] + rank
    sorted_ids = np.full(max_padded, numel, dtype=np.int32)
    sorted_ids[dest] = order.astype(np.int32)
    block_starts = np.arange(0, max_padded, block_m)
    expert_ids = np.searchsorted(padded_end, block_starts, side="right")
    expert_ids = np.where(expert_ids >= num_experts, -1, expert_ids).astype(np.int32)
    total = np.array([padded_end[-1] if nb else 0], dtype=np.int32)
    return sorted_ids, expert_ids, total


def silu_and_mul_reference(gate, up):
    s = F.silu(gate.float()).to(gate.dtype).float()
    return (s * up.float()).to(gate.dtype)


def add_rmsnorm_reference(rows, top_k, residual, weight, eps):
    """rows [T*k, H] (k = 1: x [T, H]); residual [T, H] or None. Returns (out, new_residual)."""
    H = rows.shape[-1]
    r = rows.reshape(-1, top_k, H).float()
    s = r[:, 0]
    for j in range(1, top_k):           # slot order, fp32, one rounding at the end
        s = s + r[:, j]
    x = s.to(torch.bfloat16)
    res = x if residual is None else (residual.reshape(-1, H) + x)   # bf16 add (serve.py:1192)
    xf = res.float()
    out = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float())
    return out.to(torch.bfloat16), res


def per_token_fp64(x, w13, w2, topk_weights, topk_ids):
    """sum_k w_k * W2_e(silu(W1_e x) * W3_e x) per token, float64, no intermediate rounding."""
    x = x.double()
    w13 = w13.double()
    w2 = w2.double()
    I = w2.shape[-1]
    T, H = x.shape
    out = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        for s in range(topk_ids.shape[1]):
            e = int(topk_ids[t, s])
            if e < 0 or e >= w13.shape[0]:
                continue
            g = w13[e, :I] @ x[t]
            u = w13[e, I:] @ x[t]
            a = g / (1.0 + torch.exp(-g)) * u
            out[t] += float(topk_weights[t, s]) * (w2[e] @ a)
    return out


def make_layer(T, H, E, I, dtype, seed=0, device="cpu"):
    """Seeded synthetic layer: x ~ N(0,1), router/expert weights ~ N(0, 0.02), drawn on `device`
    with that device's generator (the draws differ between CPU and GPU generators)."""
    g = torch.Generator(device=device).manual_seed(seed)

    def draw(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g, device=device) * scale).to(dtype)

    x = draw(T, H)
    gate_w = draw(E, H, scale=0.02)
    w13 = draw(E, 2 * I, H, scale=0.02)
    w2 = draw(E, H, I, scale=0.02)
    return x, gate_w, w13, w2
