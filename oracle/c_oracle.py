"""ctypes bindings for oracle/moe_oracle.c (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

The shared library is built by `make -C oracle` (also done by __graft_entry__.build()).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_moe.so")
_lib = None


def build():
    subprocess.run(["make", "-B", "-C", _HERE, "liboracle_moe.so"], check=True,
                   stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, i64, i32, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.oracle_expf.argtypes, L.oracle_expf.restype = [f32], f32
        L.oracle_dot_ordered.argtypes, L.oracle_dot_ordered.restype = [P, P, i32, i32], f32
        L.oracle_router_logits.argtypes = [P, P, i32, i64, i32, i32, P, i32, P]
        L.oracle_router_logits.restype = None
        L.oracle_route.argtypes = [P, i64, i32, i64, i32, i32, P, P, P]
        L.oracle_route.restype = None
        L.oracle_max_padded.argtypes, L.oracle_max_padded.restype = [i64, i32, i32], i64
        L.oracle_align.argtypes = [P, i64, i32, i32, P, P, P]
        L.oracle_align.restype = None
        _lib = L
    return _lib


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def expf(x: np.ndarray) -> np.ndarray:
    f = lib().oracle_expf
    x = np.asarray(x, dtype=np.float32).ravel()
    return np.array([f(float(v)) for v in x], dtype=np.float32)


def router_logits(x: np.ndarray, gate_w: np.ndarray, bias=None, logits_bf16=False):
    """x [T,H], gate_w [E,H]: float32 arrays, or uint16 arrays holding bf16 bits."""
    assert x.dtype == gate_w.dtype and x.dtype in (np.float32, np.uint16)
    dtype = 1 if x.dtype == np.uint16 else 0
    x = np.ascontiguousarray(x)
    gate_w = np.ascontiguousarray(gate_w)
    T, H = x.shape
    E = gate_w.shape[0]
    out = np.empty((T, E), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().oracle_router_logits(_ptr(x), _ptr(gate_w), dtype, T, H, E, _ptr(b),
                               int(bool(logits_bf16)), _ptr(out))
    return out


def route(logits: np.ndarray, top_k: int, renorm: bool, expert_map=None):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    w = np.empty((T, top_k), dtype=np.float32)
    ids = np.empty((T, top_k), dtype=np.int32)
    m = None if expert_map is None else np.ascontiguousarray(expert_map, dtype=np.int64)
    lib().oracle_route(_ptr(logits), T, E, E, top_k, int(bool(renorm)), _ptr(m), _ptr(w),
                       _ptr(ids))
    return w, ids


def max_padded(numel: int, E: int, block_m: int) -> int:
    return int(lib().oracle_max_padded(numel, E, block_m))


def align(ids: np.ndarray, block_m: int, E: int):
    flat = np.ascontiguousarray(np.asarray(ids).ravel(), dtype=np.int32)
    numel = flat.size
    mp = max_padded(numel, E, block_m)
    sorted_ids = np.empty(mp, dtype=np.int32)
    expert_ids = np.empty(mp // block_m, dtype=np.int32)
    total = np.empty(1, dtype=np.int32)
    lib().oracle_align(_ptr(flat), numel, E, block_m, _ptr(sorted_ids), _ptr(expert_ids),
                       _ptr(total))
    return sorted_ids, expert_ids, total
