"""SparseMoE: the qwen3_moe feed-forward block of tinyserve (serve.py:998-1099) on the HIP op.

Same parameters, buffer and weight layout as the reference module, so checkpoint loading and the
DecoderLayer that calls `self.mlp(h)` are unchanged:
    gate        nn.Linear(H, E, bias=False)        router
    w13         [E_local, 2I, H]                   gate_proj rows, then up_proj rows
    w2          [E_local, H, I]                    down_proj
    expert_map  int64 [E]                          global id -> local id, -1 = another GPU's
`forward` runs the fused router (gate GEMM + fp32 softmax/top-k/renormalise) and the experts
(align, gate_up+SwiGLU, down, k-sum). With `router="linear"` it instead computes the
logits with self.gate (bf16, as the reference does) and routes them with moe_route.
With `packed=True` (default) the experts run on an MFMA-tiled copy of w13/w2 (pack_moe_weights),
made on the first forward after the parameters change (call `pack()` before HIP-graph capture).
Changes are detected through the parameters' version counters, which in-place writes to the
parameters or their views bump; after writing through `.data`, call `pack(force=True)`.
Tensor parallelism is not part of this build: the result is this GPU's share (what the reference
passes to tp_all_reduce).
"""
import torch
from torch import nn

from . import ops


class SparseMoE(nn.Module):
    def __init__(self, cfg, router: str = "fused", packed: bool = True):
        super().__init__()
        E, H, I = cfg.num_experts, cfg.hidden_size, cfg.moe_intermediate_size
        self.top_k = cfg.num_experts_per_tok
        self.norm_topk_prob = getattr(cfg, "norm_topk_prob", True)
        self.gate = nn.Linear(H, E, bias=False)
        self.first_expert, self.num_local = getattr(cfg, "local_experts", (0, E))
        self.expert_parallel = self.num_local < E
        self.w13 = nn.Parameter(torch.empty(self.num_local, 2 * I, H))
        self.w2 = nn.Parameter(torch.empty(self.num_local, H, I))
        expert_map = torch.full((E,), -1, dtype=torch.long)
        expert_map[self.first_expert:self.first_expert + self.num_local] = torch.arange(
            self.num_local)
        self.register_buffer("expert_map", expert_map, persistent=False)
        if router not in ("fused", "linear"):
            raise ValueError("router must be 'fused' or 'linear'")
        self.router = router
        self.packed = packed
        self._packed_key = None
        self._w13_packed = None
        self._w2_packed = None

    def pack(self, force: bool = False):
        """(Re)build the MFMA-tiled weight copies if w13/w2 changed since the last pack."""
        key = (self.w13.data_ptr(), self.w2.data_ptr(), self.w13._version, self.w2._version)
        if force or key != self._packed_key:
            with torch.no_grad():
                self._w13_packed, self._w2_packed = ops.pack_moe_weights(self.w13, self.w2)
            self._packed_key = key
        return self._w13_packed, self._w2_packed

    def load_expert(self, expert: int, proj: str, fh, key: str, rank: int = 0,
                    tp: int = 1) -> bool:
        """Copy checkpoint tensor experts.{expert}.{proj}.weight into the stacked weights
        (serve.py:1052-1074). Whole experts only (expert parallel or a single GPU)."""
        e = expert - self.first_expert
        if not 0 <= e < self.num_local:
            return False
        if tp > 1 and not self.expert_parallel:
            raise NotImplementedError("TP-sliced experts are not part of this single-GPU build")
        w = fh.get_tensor(key)
        I = self.w2.shape[-1]
        with torch.no_grad():
            if proj == "gate_proj":
                self.w13[e, :I].copy_(w)
            elif proj == "up_proj":
                self.w13[e, I:].copy_(w)
            else:
                self.w2[e].copy_(w)
        return True

    def forward(self, x):
        if self.packed:
            w13, w2 = self.pack()
            if self.router == "fused":
                return ops.moe_forward_packed(x, self.gate.weight, w13, w2, self.top_k,
                                              self.norm_topk_prob, self.expert_map)
            topk_weights, topk_ids = ops.moe_route(self.gate(x), self.top_k,
                                                   self.norm_topk_prob, self.expert_map)
            return ops.fused_moe_packed(x, w13, w2, topk_weights, topk_ids)
        if self.router == "fused":
            return ops.moe_forward(x, self.gate.weight, self.w13, self.w2, self.top_k,
                                   self.norm_topk_prob, self.expert_map)
        topk_weights, topk_ids = ops.moe_route(self.gate(x), self.top_k, self.norm_topk_prob,
                                               self.expert_map)
        return ops.fused_moe(x, self.w13, self.w2, topk_weights, topk_ids)
