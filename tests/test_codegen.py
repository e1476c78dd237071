"""Properties of the compiled tile kernels that parity tests cannot see (CPU: hipcc only).

The persistent tile kernels keep their global->LDS ring in flight by hand-counted vmcnt waits. A
register spill inside the stage loop breaks that: the compiler follows every spill reload with
a wait for *all* outstanding vector-memory operations (s_waitcnt vmcnt(0)), which drains the
ring each stage. Results stay correct and only the speed suffers, so this is checked on the
gfx950 assembly of the build's own source. A stage loop is a loop nested in the per-tile loop
(depth >= 2 in the compiler's loop annotations)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tinyserve_amd", "csrc", "moe_tile.hip")


def _assembly():
    from tinyserve_amd.build import HIPCC_FLAGS, _hipcc
    flags = [f for f in HIPCC_FLAGS if f not in ("-fPIC",)]
    r = subprocess.run([_hipcc(), *flags, f"-I{os.path.dirname(SRC)}", "--offload-device-only",
                        "-S", SRC, "-o", "-"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stdout


def _stage_loop_scratch(asm: str):
    """{kernel: (scratch ops anywhere, scratch ops inside stage loops)}"""
    stats, kern, depth = {}, None, 0
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S*moe_tile_kernel\S*):", line)
        if m:
            kern = m.group(1)
            stats[kern] = [0, 0]
            depth = 0
            continue
        if kern is None:
            continue
        if re.match(r"^\.LBB\d+_\d+:", line) or "Loop Header" in line:
            d = re.search(r"Depth=(\d+)", line)
            depth = int(d.group(1)) if d else 0
        if "scratch_load" in line or "scratch_store" in line:
            stats[kern][0] += 1
            stats[kern][1] += depth >= 2
    return stats


@pytest.fixture(scope="module")
def stats():
    try:
        from tinyserve_amd.build import _hipcc
        _hipcc()
    except RuntimeError as e:
        pytest.skip(str(e))
    return _stage_loop_scratch(_assembly())


def test_every_tile_kernel_found(stats):
    heights = {re.search(r"kernelILi(\d+)E", k).group(1) for k in stats}
    assert heights == {"64", "128", "256"}, sorted(stats)
    assert len(stats) == 6  # three heights x (gate_up, down)


def test_no_spills_in_stage_loops(stats):
    bad = {k: v for k, v in stats.items() if v[1]}
    assert not bad, f"scratch accesses inside stage loops: {bad}"


def test_64_and_128_row_kernels_do_not_spill_at_all(stats):
    bad = {k: v for k, v in stats.items() if "kernelILi256E" not in k and v[0]}
    assert not bad, bad
