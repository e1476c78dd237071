"""SparseMoE: the qwen3_moe feed-forward block of tinyserve (serve.py:998-1099) on the HIP op.

Same parameters, buffer and weight layout as the reference module, so checkpoint loading and the
DecoderLayer that calls `self.mlp(h)` are unchanged:
    gate        nn.Linear(H, E, bias=False)        router
    w13         [E_local, 2I, H]                   gate_proj rows, then up_proj rows
    w2          [E_local, H, I]                    down_proj
    expert_map  int64 [E]                          global id -> local id, -1 = another GPU's
(I is this GPU's share under TP-MoE: the reference's shard_config divides moe_intermediate_size
by the tensor-parallel size, serve.py:720-725, and load_expert reads the matching slice.)

`forward` runs the fused router (gate GEMM + fp32 softmax/top-k/renormalise) and the experts
(align, gate_up+SwiGLU, down, k-sum). With `router="linear"` it instead computes the logits with
self.gate and routes them with moe_route, as the reference does. `router_logits` says what the
softmax sees in the fused mode: "model" (default) rounds the fp32-accumulated logits to the gate
weight's dtype, as the reference's nn.Linear output is (bf16 for a bf16 model, serve.py:1079);
"fp32" keeps them in fp32.

With `packed=True` (default) the experts run on the MFMA-tiled layout (pack_moe_weights), which
replaces the reference layout inside w13/w2 on the first forward (or at `pack()`), so the module
holds one copy of its expert weights. Shapes the kernels do not take as they are (e.g. I = 96, the
one-GPU share of TP-8 for Qwen3-30B-A3B) are zero-padded there (ops.padded_shape), which changes
the parameters' shapes while packed. The module hands its weights back in the reference layout
wherever they leave or enter it: `state_dict()` returns reference-layout tensors,
`load_state_dict()` and `load_expert()` first restore the reference layout (`unpack()`), and the
next forward packs again. Writing into w13/w2 directly while they hold the packed layout is an
error that forward reports; call `unpack()` first (or, after writing reference-layout values
into the packed-shape tensors through `.data`, `pack(force=True)`).
Tensor parallelism is not part of this build: the result is this GPU's share (what the reference
passes to tp_all_reduce).
"""
import torch
from torch import nn

from . import layout, ops

ROUTER_LOGITS = ("model", "fp32")


def load_shard(fh, key: str, rank: int, tp: int) -> torch.Tensor:
    """This rank's slice of an expert tensor under TP-MoE (the rule of serve.py:731-777 for the
    expert projections): gate_proj / up_proj are split along their output rows, down_proj along
    its input columns. tp == 1 reads the whole tensor."""
    if tp == 1:
        return fh.get_tensor(key)
    sl = fh.get_slice(key)
    rows, cols = sl.get_shape()
    if "down_proj" in key:
        n = cols // tp
        return sl[:, rank * n:(rank + 1) * n]
    n = rows // tp
    return sl[rank * n:(rank + 1) * n]


class SparseMoE(nn.Module):
    def __init__(self, cfg, router: str = "fused", packed: bool = True,
                 router_logits: str = "model"):
        super().__init__()
        E, H, I = cfg.num_experts, cfg.hidden_size, cfg.moe_intermediate_size
        self.top_k = cfg.num_experts_per_tok
        self.norm_topk_prob = getattr(cfg, "norm_topk_prob", True)
        self.gate = nn.Linear(H, E, bias=False)
        self.first_expert, self.num_local = getattr(cfg, "local_experts", (0, E))
        self.expert_parallel = self.num_local < E
        self.hidden_size, self.intermediate_size = H, I
        self.w13 = nn.Parameter(torch.empty(self.num_local, 2 * I, H))
        self.w2 = nn.Parameter(torch.empty(self.num_local, H, I))
        expert_map = torch.full((E,), -1, dtype=torch.long)
        expert_map[self.first_expert:self.first_expert + self.num_local] = torch.arange(
            self.num_local)
        self.register_buffer("expert_map", expert_map, persistent=False)
        if router not in ("fused", "linear"):
            raise ValueError("router must be 'fused' or 'linear'")
        if router_logits not in ROUTER_LOGITS:
            raise ValueError(f"router_logits must be one of {ROUTER_LOGITS}")
        self.router = router
        self.router_logits = router_logits
        self.packed = packed
        self.weights_packed = False   # True while w13/w2 hold the MFMA-tiled layout
        self._packed_key = None
        self._register_state_dict_hook(SparseMoE._reference_layout_state)
        self._register_load_state_dict_pre_hook(SparseMoE._before_load, with_module=True)

    # ---- layout management
    def _key(self):
        return (self.w13.data_ptr(), self.w2.data_ptr(), self.w13._version, self.w2._version)

    def pack(self, force: bool = False):
        """Replace the reference-layout w13/w2 by their MFMA-tiled (packed) layout, in place. A
        no-op when already packed, unless `force` (the parameters then hold reference-layout
        values of the packed shape, written through `.data`). Call it before HIP-graph capture.
        Returns the packed (w13, w2)."""
        if self.weights_packed and not force:
            self._check_untouched()
            return self.w13, self.w2
        with torch.no_grad():
            if self.weights_packed:   # force: reference values in the packed-shape tensors
                w13, w2 = self._ref_view()
            else:
                w13, w2 = self.w13, self.w2
            p13, p2 = ops.pack_moe_weights(w13.contiguous(), w2.contiguous())
            del w13, w2
            self.w13.data = p13
            self.w2.data = p2
        self.weights_packed = True
        self._packed_key = self._key()
        return self.w13, self.w2

    def _ref_view(self):
        """Reference-layout views into parameters that hold reference values in a (possibly
        padded) packed-shape tensor (the `pack(force=True)` case)."""
        I, H = self.intermediate_size, self.hidden_size
        Ip = self.w13.shape[1] // 2
        w13 = torch.cat([self.w13[:, :I, :H], self.w13[:, Ip:Ip + I, :H]], 1)
        return w13, self.w2[:, :H, :I]

    def unpack(self):
        """Restore the reference layout (and shapes) of w13/w2 in place."""
        if not self.weights_packed:
            return
        self._check_untouched()
        with torch.no_grad():
            I, H = self.intermediate_size, self.hidden_size
            w13 = layout.unpack(self.w13.data, True, 2 * I, H)
            w2 = layout.unpack(self.w2.data, False, H, I)
            self.w13.data = w13
            self.w2.data = w2
        self.weights_packed = False
        self._packed_key = None

    def _check_untouched(self):
        if self._packed_key is not None and self._key() != self._packed_key:
            raise RuntimeError(
                "SparseMoE: w13/w2 were written while holding the packed layout; call unpack() "
                "before writing reference-layout weights (load_expert and load_state_dict do)")

    def _apply(self, fn, *args, **kwargs):
        # moving or casting the module keeps the packed contents; re-key on the new tensors
        out = super()._apply(fn, *args, **kwargs)
        if self.weights_packed:
            self._packed_key = self._key()
        return out

    @staticmethod
    def _reference_layout_state(module, state, prefix, local_metadata):
        if module.weights_packed:
            I, H = module.intermediate_size, module.hidden_size
            with torch.no_grad():
                state[prefix + "w13"] = layout.unpack(module.w13.detach(), True, 2 * I, H)
                state[prefix + "w2"] = layout.unpack(module.w2.detach(), False, H, I)
        return state

    def _before_load(self, state_dict, prefix, *args, **kwargs):
        self.unpack()

    # ---- checkpoint loading
    def load_expert(self, expert: int, proj: str, fh, key: str, rank: int = 0,
                    tp: int = 1) -> bool:
        """Copy checkpoint tensor experts.{expert}.{proj}.weight into the stacked weights
        (serve.py:1052-1074): whole experts under expert parallelism, else this rank's TP-MoE
        slice (load_shard)."""
        e = expert - self.first_expert
        if not 0 <= e < self.num_local:
            return False
        self.unpack()
        w = fh.get_tensor(key) if self.expert_parallel else load_shard(fh, key, rank, tp)
        I = self.w2.shape[-1]
        with torch.no_grad():
            if proj == "gate_proj":
                self.w13[e, :I].copy_(w)
            elif proj == "up_proj":
                self.w13[e, I:].copy_(w)
            else:
                self.w2[e].copy_(w)
        return True

    # ---- forward
    def _logits_bf16(self):
        return self.router_logits == "model" and self.gate.weight.dtype == torch.bfloat16

    def rows(self, x):
        """The block's per-slot rows [T * top_k, H] (row t*k + s = routing weight x expert output
        of token t's slot s), unsummed: the reference's fused_moe(..., sum_topk=False)
        (serve.py:1084-1085), for a caller that fuses the k-sum into what follows
        (ops.moe_combine_add_rmsnorm)."""
        return self.forward(x, sum_topk=False)

    def forward(self, x, sum_topk: bool = True):
        # the packed layout is for the bf16 matrix-core kernels; fp32 layers run unpacked
        if self.packed and (self.weights_packed or self.w13.dtype == torch.bfloat16):
            w13, w2 = self.pack()
            if self.router == "fused":
                return ops.moe_forward_packed(x, self.gate.weight, w13, w2, self.top_k,
                                              self.norm_topk_prob, self.expert_map, None,
                                              self._logits_bf16(), sum_topk)
            topk_weights, topk_ids = ops.moe_route(self.gate(x), self.top_k,
                                                   self.norm_topk_prob, self.expert_map)
            return ops.fused_moe_packed(x, w13, w2, topk_weights, topk_ids, sum_topk)
        self.unpack()
        if self.router == "fused":
            return ops.moe_forward(x, self.gate.weight, self.w13, self.w2, self.top_k,
                                   self.norm_topk_prob, self.expert_map, None,
                                   self._logits_bf16(), sum_topk)
        topk_weights, topk_ids = ops.moe_route(self.gate(x), self.top_k, self.norm_topk_prob,
                                               self.expert_map)
        return ops.fused_moe(x, self.w13, self.w2, topk_weights, topk_ids, sum_topk)
