"""Loads libtinyserve_moe.so and declares the C ABI of include/tinyserve_moe.h for ctypes.

torch is imported first so that the library binds to the HIP runtime torch already loaded (one
runtime per process: torch's streams and the library's launches then share the same queues).
There is no fallback: if the library is missing the import fails.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtinyserve_moe.so")

TSM_F32, TSM_BF16 = 0, 1


class TsmError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


P, I64, I32, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
# argument and result types of every entry point of include/tinyserve_moe.h
SIGNATURES = {
    "tsm_last_error": ([], ctypes.c_char_p),
    "tsm_abi_version": ([], I32),
    "tsm_moe_route": ([P, I32, I64, I32, I64, I32, I32, P, P, P, P], I32),
    "tsm_moe_router": ([P, P, I32, I64, I32, I32, I32, I32, P, P, I32, P, P, P, P], I32),
    "tsm_moe_max_padded": ([I64, I32, I32], I64),
    "tsm_moe_align_workspace_size": ([I64, I32, I32], SZ),
    "tsm_moe_align": ([P, I64, I32, I32, P, P, P, P, SZ, P], I32),
    "tsm_silu_and_mul": ([P, I64, P, I64, P, I64, I64, I64, P], I32),
    "tsm_moe_block_m": ([I64, I32, I32, I32, I32, I32], I32),
    "tsm_moe_set_block_m": ([I64, I64, I32, I32], I32),
    "tsm_fused_moe_workspace_size": ([I64, I32, I32, I32, I32], SZ),
    "tsm_fused_moe": ([P, P, P, P, P, I64, I32, I32, I32, I32, I32, P, P, SZ, P], I32),
    "tsm_fused_moe_f32_workspace_size": ([I64, I32, I32, I32, I32], SZ),
    "tsm_fused_moe_f32": ([P, P, P, P, P, I64, I32, I32, I32, I32, I32, P, P, SZ, P], I32),
    "tsm_moe_gemm_gate_up": ([P, P, P, P, P, I64, I32, I32, I32, I32, I32, I32, P, P], I32),
    "tsm_moe_gemm_down": ([P, P, P, P, P, P, I64, I32, I32, I32, I32, I32, P, P], I32),
    "tsm_moe_expert_gate_up": ([P, P, P, I64, I32, I32, I32, I32, I32, P, P], I32),
    "tsm_moe_expert_down": ([P, P, P, P, I64, I32, I32, I32, I32, P, P], I32),
    "tsm_moe_pack_weights": ([P, I64, I32, I32, I32, P, P], I32),
    "tsm_moe_padded_shape": ([I32, I32, P, P], I32),
    "tsm_moe_pack_weights_padded": ([P, I64, I32, I32, I32, I32, I32, P, P], I32),
    "tsm_fused_moe_packed": ([P, P, P, P, P, I64, I32, I32, I32, I32, I32, P, P, SZ, P], I32),
    "tsm_moe_forward_packed": ([P, P, P, P, P, P, I64, I32, I32, I32, I32, I32, I32, I32, P, P,
                                P, P, SZ, P], I32),
    "tsm_moe_combine": ([P, I64, I32, I32, P, P], I32),
    "tsm_qk_norm_rope": ([P, I64, I32, I64, I64, P, I32, I64, I64, P, I64, I64, I32, P, P, I64,
                          P, P, ctypes.c_float, P, P, I64, I32, P, P], I32),
    "tsm_paged_attention": ([P, I64, I32, I64, I64, P, P, I64, I32, I32, I32, P, P, P, I64,
                             I32, I32, ctypes.c_float, I32, P, SZ, P, I64, I64, P], I32),
    "tsm_paged_attention_workspace_size": ([I32, I32, I32, I32], SZ),
    "tsm_greedy_argmax": ([P, I32, I64, I64, I32, P, P], I32),
    "tsm_add_rmsnorm": ([P, I64, I32, I32, P, I32, P, ctypes.c_float, P, P], I32),
    "tsm_moe_forward_workspace_size": ([I64, I32, I32, I32, I32], SZ),
    "tsm_moe_forward": ([P, P, P, P, P, P, I64, I32, I32, I32, I32, I32, I32, I32, P, P, P,
                         P, SZ, P], I32),
}


def bind(L):
    """Declare the C ABI's argument and result types on a loaded library."""
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    return L


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python tinyserve_amd/build.py` "
            "(or __graft_entry__.build()); tinyserve_amd has no non-HIP fallback")
    return bind(ctypes.CDLL(LIB_PATH))


lib = _load()


def check(rc: int, what: str):
    if rc != 0:
        msg = lib.tsm_last_error().decode(errors="replace")
        raise TsmError(f"{what} failed (status {rc}): {msg}")


def ptr(t):
    """Device pointer of a tensor (or None)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
