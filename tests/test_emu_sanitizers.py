"""The CPU-emulated kernels under sanitizers, in child processes with the sanitizer's runtime
preloaded; each runs a subset of test_emu_kernels.py (the quick cases: each kernel family and
plan at least once). Both children run at once.

- AddressSanitizer + UndefinedBehaviorSanitizer: every memory access the kernels make (global
  memory, LDS, the global->LDS loads) is checked, so an index past a buffer fails here, on the
  CPU, instead of faulting a GPU.
- ThreadSanitizer: each wavefront is a sanitizer fiber, and the only ordering between them is
  what the GPU guarantees (barriers and kernel boundaries), so two wavefronts touching the same
  LDS or global bytes between barriers, or two workgroups of a launch writing the same bytes,
  are reported as data races.

A whole file under one of them: `TSM_EMU_SANITIZER=asan LD_PRELOAD=<libclang_rt.asan> python -m
pytest -s tests/test_emu_kernels.py` (tsan likewise, with TSAN_OPTIONS=halt_on_error=1)."""
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "emu"))

import build_emu  # noqa: E402
import harness  # noqa: E402

QUICK = "not end_to_end and not autotune and not every_plan or every_plan and 2"
SANITIZERS = ["asan", "tsan"]


@pytest.fixture(scope="module")
def children():
    """Builds both libraries (each build is itself parallel), then starts both runs."""
    running = {}
    for san in SANITIZERS:
        if harness.sanitizer_runtime(san) is not None:
            build_emu.build(san)
    for san in SANITIZERS:
        if harness.sanitizer_runtime(san) is not None:
            running[san] = harness.start_under_sanitizer("tests/test_emu_kernels.py", san,
                                                         select=QUICK)
    yield running
    for proc, out in running.values():
        if proc.poll() is None:
            proc.kill()
            proc.wait()
        out.close()


@pytest.mark.parametrize("sanitizer", SANITIZERS)
def test_kernels_under_sanitizer(children, sanitizer):
    if sanitizer not in children:
        pytest.skip(f"no {sanitizer} runtime in this toolchain")
    rc, report = harness.finish(*children[sanitizer], timeout=1200)
    assert rc == 0, report
    for marker in ("ERROR: AddressSanitizer", "runtime error", "WARNING: ThreadSanitizer"):
        assert marker not in report, report
