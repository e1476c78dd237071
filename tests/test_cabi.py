"""CPU tests of the C ABI: the library loads, exports every symbol declared in
include/tinyserve_moe.h, and its size/validation entry points behave (no kernel launches)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tinyserve_moe.h")
LIB = os.path.join(ROOT, "tinyserve_amd", "libtinyserve_moe.so")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(tsm_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail("libtinyserve_moe.so not built (run __graft_entry__.build())")
    import torch  # noqa: F401  (same load order as the package)
    return ctypes.CDLL(LIB)


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n


def test_package_signatures_cover_header():
    import tinyserve_amd._lib as L
    src = open(L.__file__).read()
    for n in declared():
        assert f'"{n}"' in src, n


def test_sizes(lib):
    lib.tsm_moe_max_padded.restype = ctypes.c_int64
    lib.tsm_moe_max_padded.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int]
    assert lib.tsm_moe_max_padded(512, 128, 16) == 2448       # T=64 decode
    assert lib.tsm_moe_max_padded(65536, 128, 64) == 73664    # T=8192 prefill
    assert lib.tsm_moe_max_padded(4, 3, 4) == 16              # docstring example
    lib.tsm_fused_moe_workspace_size.restype = ctypes.c_size_t
    lib.tsm_fused_moe_workspace_size.argtypes = [ctypes.c_int64] + [ctypes.c_int] * 4
    # T=64 runs expert-major (compact activations, one row per assignment) plus the per-slot rows
    assert lib.tsm_fused_moe_workspace_size(64, 2048, 768, 128, 8) >= 512 * (768 + 2048) * 2
    # T=8192 runs the tiled path: activations for every padded row
    assert lib.tsm_fused_moe_workspace_size(8192, 2048, 768, 128, 8) >= 73664 * 768 * 2
    lib.tsm_abi_version.restype = ctypes.c_int
    assert lib.tsm_abi_version() == 1


def test_invalid_arguments_return_codes(lib):
    """Validation happens before any HIP call, so these run without a GPU."""
    P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.tsm_last_error.restype = ctypes.c_char_p
    f = lib.tsm_moe_route
    f.argtypes = [P, I32, I64, I32, I64, I32, I32, P, P, P, P]
    assert f(None, 0, 4, 128, 128, 0, 1, None, None, None, None) == -1          # top_k = 0
    assert b"top_k" in lib.tsm_last_error()
    assert f(None, 0, 4, 1000, 1000, 8, 1, None, None, None, None) == -2        # E > 512
    assert f(None, 7, 4, 128, 128, 8, 1, None, P(16), P(16), P(16)) == -1       # null logits
    g = lib.tsm_fused_moe
    g.argtypes = [P, P, P, P, P, I64, I32, I32, I32, I32, I32, P, P, ctypes.c_size_t, P]
    assert g(P(256), P(256), P(256), P(256), P(256), 4, 100, 768, 128, 8, 1, P(256), P(256),
             1 << 30, None) == -2                                                # H % 128
    assert g(P(256), P(256), P(256), P(256), P(256), 4, 2048, 768, 128, 8, 1, P(256), P(256),
             16, None) == -4                                                     # workspace
    assert b"workspace" in lib.tsm_last_error()
    assert g(None, None, None, None, None, 0, 2048, 768, 128, 8, 1, None, None, 0, None) == 0


def test_padded_shape_and_norm_validation(lib):
    P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.tsm_last_error.restype = ctypes.c_char_p
    ps = lib.tsm_moe_padded_shape
    ps.argtypes = [I32, I32, P, P]
    hp, ip = ctypes.c_int(), ctypes.c_int()
    for (H, I), want in {(2048, 768): (2048, 768), (2048, 96): (2048, 128),
                         (200, 50): (256, 128), (2048, 192): (2048, 192)}.items():
        assert ps(H, I, ctypes.byref(hp), ctypes.byref(ip)) == 0
        assert (hp.value, ip.value) == want
    assert ps(0, 96, ctypes.byref(hp), ctypes.byref(ip)) == -1
    pk = lib.tsm_moe_pack_weights_padded
    pk.argtypes = [P, I64, I32, I32, I32, I32, I32, P, P]
    assert pk(P(256), 2, 192, 2048, 200, 2048, 1, P(512), None) == -2   # N_pad % 32 (interleaved)
    assert pk(P(256), 2, 192, 2048, 128, 2048, 1, P(512), None) == -2   # N_pad < N
    assert pk(P(256), 2, 2048, 96, 2048, 100, 0, P(512), None) == -2    # K_pad % 32
    assert pk(P(256), 2, 2048, 96, 2048, 128, 0, P(256), None) == -1    # in place
    nf = lib.tsm_add_rmsnorm
    nf.argtypes = [P, I64, I32, I32, P, I32, P, ctypes.c_float, P, P]
    assert nf(P(256), 4, 100, 1, None, 0, P(256), 1e-6, P(512), None) == -2     # H % 8
    assert nf(P(256), 4, 32768, 1, None, 0, P(256), 1e-6, P(512), None) == -2   # H too large
    assert nf(P(256), 4, 2048, 0, None, 0, P(256), 1e-6, P(512), None) == -1    # top_k
    assert nf(P(256), 4, 2048, 8, None, 1, P(256), 1e-6, P(512), None) == -1    # no residual
    assert b"residual" in lib.tsm_last_error()
    assert nf(None, 4, 2048, 8, None, 0, P(256), 1e-6, P(512), None) == -1      # null x
    assert nf(None, 0, 2048, 8, None, 0, None, 1e-6, None, None) == 0           # empty batch


def test_plan_overrides(lib):
    """Installed tile heights change the plan (and the workspace follows); -1 restores it."""
    I32, I64 = ctypes.c_int, ctypes.c_int64
    lib.tsm_moe_set_block_m.argtypes = [I64, I64, I32, I32]
    lib.tsm_moe_block_m.argtypes = [I64, I32, I32, I32, I32, I32]
    ws = lib.tsm_fused_moe_workspace_size
    ws.restype = ctypes.c_size_t
    ws.argtypes = [I64, I32, I32, I32, I32]
    base = lib.tsm_moe_block_m(64, 2048, 768, 128, 8, 0)
    assert base == 0                                        # expert-major at T=64
    w0 = ws(64, 2048, 768, 128, 8)
    assert lib.tsm_moe_set_block_m(512, 512, 0, 64) == 0
    assert lib.tsm_moe_block_m(64, 2048, 768, 128, 8, 0) == 64
    assert lib.tsm_moe_block_m(64, 2048, 768, 128, 8, 1) == 0   # the other layout untouched
    assert ws(64, 2048, 768, 128, 8) > w0                   # padded rows for 64-row tiles
    assert lib.tsm_moe_set_block_m(512, 512, 0, 128) == -2  # no 128-row reference kernel
    assert lib.tsm_moe_set_block_m(512, 512, 1, 128) == 0
    assert lib.tsm_moe_block_m(64, 2048, 768, 128, 8, 1) == 128
    assert lib.tsm_moe_set_block_m(1, 1 << 40, 0, -1) == 0
    assert lib.tsm_moe_set_block_m(1, 1 << 40, 1, -1) == 0
    assert lib.tsm_moe_block_m(64, 2048, 768, 128, 8, 0) == base
    assert lib.tsm_moe_set_block_m(0, 4, 0, 16) == -1       # numel_lo >= 1


def test_attention_validation(lib):
    """Head counts are checked before they are divided (a host-side UBSan run found H = 0
    reaching a modulo by zero)."""
    P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    f = lib.tsm_paged_attention
    f.argtypes = [P, I64, I32, I64, I64, P, P, I64, I32, I32, I32, P, P, P, I64, I32, I32,
                  ctypes.c_float, I32, P, ctypes.c_size_t, P, I64, I64, P]
    args = lambda H, Hkv, D=128, page=16, S=1, ws=None, nws=0: (  # noqa
        P(256), 4, H, H * D, D, P(256), P(256), 8, page, Hkv, D, P(256), P(256), P(256), 4, 2,
        1, 0.1, S, ws, nws, P(256), H * D, D, None)
    assert f(*args(0, 4)) == -1
    assert f(*args(32, 0)) == -1
    assert f(*args(2, 4)) == -1           # fewer query heads than KV heads
    assert f(*args(32 * 3, 3)) == -2      # group 32 does not divide 16
    assert f(*args(32, 4, D=96)) == -2    # head_dim
    assert f(*args(32, 4, page=6)) == -2  # page % 4
    # split-KV: split count range, and the workspace it needs
    ws = lib.tsm_paged_attention_workspace_size
    ws.argtypes, ws.restype = [I32, I32, I32, I32], ctypes.c_size_t
    assert ws(2, 32, 128, 1) == 0 and ws(2, 32, 128, 0) == 0 and ws(2, 32, 128, 65) == 0
    need = ws(2, 32, 128, 8)
    assert need == 2 * 32 * 8 * 128 * 4 + 2 * 32 * 8 * 4
    assert f(*args(32, 4, S=0)) == -1 and f(*args(32, 4, S=65)) == -1
    assert f(*args(32, 4, S=8)) == -4                                 # no workspace
    assert f(*args(32, 4, S=8, ws=P(256), nws=need - 1)) == -4        # too small
    assert f(*args(32, 4, S=8, ws=P(264), nws=need)) == -4            # not 256-byte aligned


def test_128_row_plan_only_where_the_tile_kernels_run(lib):
    I32, I64, P = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
    lib.tsm_moe_block_m.argtypes = [I64, I32, I32, I32, I32, I32]
    assert lib.tsm_moe_block_m(8192, 2048, 768, 128, 8, 1) == 128
    assert lib.tsm_moe_block_m(8192, 128, 64, 32, 8, 1) == 64      # 2I % 256 != 0
    assert lib.tsm_moe_block_m(8192, 2176, 768, 32, 8, 1) == 64    # H % 256 != 0
    lib.tsm_moe_set_block_m.argtypes = [I64, I64, I32, I32]
    assert lib.tsm_moe_set_block_m(1, 1 << 30, 1, 128) == 0
    assert lib.tsm_moe_block_m(64, 128, 64, 32, 8, 1) == 64        # installed 128 not taken
    assert lib.tsm_moe_set_block_m(1, 1 << 30, 1, -1) == 0
    f = lib.tsm_moe_gemm_gate_up
    f.argtypes = [P, P, P, P, P, I64, I32, I32, I32, I32, I32, I32, P, P]
    lib.tsm_last_error.restype = ctypes.c_char_p
    assert f(P(256), P(256), P(256), P(256), P(256), 512, 8, 128, 64, 32, 128, 1, P(256),
             None) == -2
    assert b"128-row" in lib.tsm_last_error()


def test_256_row_plan_only_below_4_gib_of_x(lib):
    """An installed 256-row plan applies only while x (T x H bf16) is below 4 GiB: the 256-row
    gate_up kernel gathers x rows through 32-bit byte offsets. Past that, the static plan."""
    I32, I64 = ctypes.c_int, ctypes.c_int64
    lib.tsm_moe_set_block_m.argtypes = [I64, I64, I32, I32]
    lib.tsm_moe_block_m.argtypes = [I64, I32, I32, I32, I32, I32]
    H, I, E, k = 2048, 768, 128, 8
    assert lib.tsm_moe_set_block_m(1, 1 << 30, 1, 256) == 0
    try:
        small = 8192
        big = (1 << 32) // (2 * H)         # the first T with 4 GiB of x
        assert lib.tsm_moe_block_m(small, H, I, E, k, 1) == 256
        assert lib.tsm_moe_block_m(big - 1, H, I, E, k, 1) == 256
        assert lib.tsm_moe_block_m(big, H, I, E, k, 1) == 128   # the static table's choice
    finally:
        assert lib.tsm_moe_set_block_m(1, 1 << 30, 1, -1) == 0
