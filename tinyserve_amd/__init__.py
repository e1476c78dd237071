"""tinyserve_amd: MI355X-native (gfx950 HIP) fused mixture-of-experts operator for tinyserve's
qwen3_moe block. Importing requires the built libtinyserve_moe.so (there is no fallback)."""
from . import checkpoint, kernels, ops  # noqa: F401
from ._lib import TsmError, lib  # noqa: F401
from .kernels import (autotune_fused_moe, fused_moe, moe_align_block_size,  # noqa: F401
                      moe_align_block_size_triton, moe_route, silu_and_mul)
from .checkpoint import load_moe_checkpoint  # noqa: F401
from .moe import SparseMoE  # noqa: F401
from .ops import (fused_moe_packed, moe_forward, moe_forward_packed, moe_router,  # noqa: F401
                  pack_moe_weights)

__all__ = ["fused_moe", "moe_route", "moe_router", "moe_forward", "moe_align_block_size",
           "moe_align_block_size_triton", "silu_and_mul", "autotune_fused_moe", "SparseMoE", "pack_moe_weights", "fused_moe_packed",
           "moe_forward_packed", "load_moe_checkpoint",
           "TsmError"]
