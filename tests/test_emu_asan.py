"""The CPU-emulated kernels under AddressSanitizer and UndefinedBehaviorSanitizer: every memory
access the kernels make (global memory, LDS, the global->LDS loads) is checked, so an index past a
buffer fails here, on the CPU, instead of faulting a GPU. Runs a subset of test_emu_kernels.py
(the quick cases: each kernel family and plan at least once) in a child process with the
sanitizer runtime preloaded; the whole file under the sanitizers is
`TSM_EMU_ASAN=1 LD_PRELOAD=<libclang_rt.asan> python -m pytest tests/test_emu_kernels.py`."""
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "emu"))

import harness  # noqa: E402


def test_kernels_under_sanitizers():
    if harness.asan_runtime() is None:
        pytest.skip("no AddressSanitizer runtime in this toolchain")
    r = harness.run_under_asan(
        "tests/test_emu_kernels.py", timeout=900,
        select="not end_to_end and not every_plan or every_plan and 2")
    report = (r.stdout + r.stderr)[-6000:]
    assert r.returncode == 0, report
    assert "ERROR: AddressSanitizer" not in report and "runtime error" not in report, report
