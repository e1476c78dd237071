"""Runs the product's Python ops on CPU tensors through the emulated kernels (TEST ONLY).

`emulated(asan=False)` is a context manager that swaps, for its duration, the library the
tinyserve_amd modules call (tinyserve_amd/libtinyserve_moe.so) for the CPU build of the same
kernel sources (tests/emu/build_emu.py), and lets the ops take CPU tensors (their device checks
and stream lookup are replaced; the tensors' host addresses are passed as the device pointers).
On exit everything is restored. The product itself never loads the emulation library.

The ASan build needs the AddressSanitizer runtime loaded first, which a running interpreter cannot
do; `run_under_asan(test_file)` starts a child pytest process with it preloaded.
"""
import contextlib
import ctypes
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

import build_emu  # noqa: E402

_LIBS = {}


def load(asan: bool = False):
    if asan not in _LIBS:
        import tinyserve_amd._lib as L
        _LIBS[asan] = L.bind(ctypes.CDLL(build_emu.build(asan=asan)))
    return _LIBS[asan]


@contextlib.contextmanager
def emulated(asan: bool = False):
    import tinyserve_amd._lib as L
    from tinyserve_amd import attention, kernels, ops
    emu = load(asan)
    saved = []

    def patch(mod, name, value):
        saved.append((mod, name, getattr(mod, name)))
        setattr(mod, name, value)

    no_check = lambda *ts: None  # noqa: E731
    patch(ops, "torch", _AlignedTorch())
    no_stream = lambda t=None: None  # noqa: E731
    for mod in (L, ops, attention, kernels):
        patch(mod, "lib", emu)
    patch(ops, "_on_gpu", no_check)
    patch(attention, "_gpu", no_check)
    patch(ops, "stream_of", no_stream)
    patch(attention, "stream_of", no_stream)
    patch(L, "stream_of", no_stream)
    import torch
    patch(torch.cuda, "synchronize", lambda *a, **k: None)
    try:
        yield emu
    finally:
        for mod, name, value in reversed(saved):
            setattr(mod, name, value)


class _AlignedTorch:
    """torch, except that 1-D uint8 buffers (the ops' workspaces) come 256-byte aligned, as the
    GPU caching allocator returns them; the CPU allocator aligns to 64 bytes."""

    def __getattr__(self, name):
        import torch
        return getattr(torch, name)

    def empty(self, *size, **kw):
        import torch
        if kw.get("dtype") == torch.uint8 and len(size) == 1 and isinstance(size[0], int):
            raw = torch.empty(size[0] + 256, **kw)
            off = (-raw.data_ptr()) % 256
            return raw[off:off + size[0]]
        return torch.empty(*size, **kw)


def asan_runtime():
    import glob
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


def run_under_asan(test_file: str, timeout: int = 900, select: str = None):
    """pytest on `test_file` (optionally `-k select`) in a child process with the ASan runtime
    preloaded and TSM_EMU_ASAN=1 (the tests then use the ASan build). Returns the
    CompletedProcess."""
    rt = asan_runtime()
    preload = " ".join(x for x in (rt, os.environ.get("LD_PRELOAD", "")) if x)
    env = dict(os.environ, TSM_EMU_ASAN="1", LD_PRELOAD=preload,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", test_file]
    if select:
        cmd += ["-k", select]
    return subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True,
                          timeout=timeout)
