"""Runs the product's Python ops on CPU tensors through the emulated kernels (TEST ONLY).

`emulated(sanitizer=None)` is a context manager that swaps, for its duration, the library the
tinyserve_amd modules call (tinyserve_amd/libtinyserve_moe.so) for the CPU build of the same
kernel sources (tests/emu/build_emu.py), and lets the ops take CPU tensors (their device checks
and stream lookup are replaced; the tensors' host addresses are passed as the device pointers).
On exit everything is restored. The product itself never loads the emulation library.

The sanitizer builds ("asan": AddressSanitizer + UBSan, out-of-bounds accesses; "tsan":
ThreadSanitizer, data races between wavefronts and workgroups) need their runtime loaded first,
which a running interpreter cannot do; `start_under_sanitizer(test_file, sanitizer)` starts a child
pytest process with it preloaded and TSM_EMU_SANITIZER set, which the emulated tests and
`pytest --emulate` read to pick the build.
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


def load(sanitizer: str = None):
    if sanitizer not in _LIBS:
        import tinyserve_amd._lib as L
        _LIBS[sanitizer] = L.bind(ctypes.CDLL(build_emu.build(sanitizer)))
    return _LIBS[sanitizer]


def sanitizer_from_env():
    """The build the current process was started for (TSM_EMU_SANITIZER: asan, tsan or unset)."""
    return os.environ.get("TSM_EMU_SANITIZER") or None


@contextlib.contextmanager
def emulated(sanitizer: str = None):
    import tinyserve_amd._lib as L
    from tinyserve_amd import attention, kernels, ops
    emu = load(sanitizer)
    saved = []

    def patch(mod, name, value):
        saved.append((mod, name, getattr(mod, name)))
        setattr(mod, name, value)

    no_check = lambda *ts: None  # noqa: E731
    patch(ops, "torch", _AlignedTorch())
    patch(attention, "torch", _AlignedTorch())
    # the split-KV choice asks for the device's CU count: the emulated device has MI355X's 256
    choose = attention.choose_num_splits
    patch(attention, "choose_num_splits",
          lambda programs, max_seq_len, device: choose(programs, max_seq_len, "cuda:0"))
    patch(attention, "_cu_counts", {0: 256})
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
    patch(torch.cuda, "Event", _HostEvent)   # timing code (autotuning) runs on the host clock
    try:
        yield emu
    finally:
        for mod, name, value in reversed(saved):
            setattr(mod, name, value)


class _HostEvent:
    """torch.cuda.Event stand-in: the emulated kernels run synchronously, so an event is
    complete when recorded and the host clock times them."""

    def __init__(self, enable_timing=False, **_):
        self.t = None

    def record(self, stream=None):
        import time
        self.t = time.perf_counter()

    def synchronize(self):
        pass

    def query(self):
        return True

    def elapsed_time(self, end):
        return (end.t - self.t) * 1e3


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


def sanitizer_runtime(sanitizer: str):
    import glob
    found = sorted(glob.glob(
        f"/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.{sanitizer}-x86_64.so"))
    return found[-1] if found else None


SANITIZER_ENV = {
    "asan": {"ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=1",
             "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"},
    # one intra-op thread: torch's own worker threads are not part of what is checked
    "tsan": {"TSAN_OPTIONS": "halt_on_error=1:report_signal_unsafe=0:history_size=4",
             "OMP_NUM_THREADS": "1"},
}


def start_under_sanitizer(test_file: str, sanitizer: str, select: str = None):
    """Starts pytest on `test_file` (optionally `-k select`) in a child process with the
    sanitizer's runtime preloaded and TSM_EMU_SANITIZER set (the emulated tests then use that
    build); its output goes to a temporary file. Returns (Popen, output file)."""
    import tempfile
    rt = sanitizer_runtime(sanitizer)
    preload = " ".join(x for x in (rt, os.environ.get("LD_PRELOAD", "")) if x)
    env = dict(os.environ, TSM_EMU_SANITIZER=sanitizer, LD_PRELOAD=preload,
               **SANITIZER_ENV[sanitizer])
    # -s: a sanitizer report that ends the process goes straight to the output file
    cmd = [sys.executable, "-m", "pytest", "-x", "-q", "-s", "-p", "no:cacheprovider", test_file]
    if select:
        cmd += ["-k", select]
    out = tempfile.TemporaryFile(mode="w+")
    return subprocess.Popen(cmd, cwd=ROOT, env=env, stdout=out, stderr=subprocess.STDOUT,
                            text=True), out


def finish(proc, out, timeout: int):
    """Waits for a child started by start_under_sanitizer; returns (returncode, output tail)."""
    try:
        rc = proc.wait(timeout=timeout)
    except subprocess.TimeoutExpired:
        proc.kill()
        proc.wait()
        rc = "timeout"
    out.seek(0)
    return rc, out.read()[-8000:]
