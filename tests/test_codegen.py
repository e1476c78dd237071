"""Properties of the compiled tile kernels that parity tests cannot see (CPU: hipcc only).

The persistent tile kernels keep their global->LDS ring in flight by hand-counted vmcnt waits. A
register spill inside the stage loop breaks that: the compiler follows every spill reload with
a wait for *all* outstanding vector-memory operations (s_waitcnt vmcnt(0)), which drains the
ring each stage. Results stay correct and only the speed suffers, so this is checked on the
gfx950 assembly of the build's own source. A stage loop is a loop nested in the per-tile loop
(depth >= 2 in the compiler's loop annotations).

The prefill (128- and 256-row) kernels' stage loops are also checked for LDS latency: every fragment read there is
consumed only several MFMAs after it issues (each 16x16x32 MFMA occupies a SIMD for about 16
cycles at the dense rate, so 6 MFMAs cover the LDS read latency), including reads consumed in
the next iteration."""
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


def _regs(spec):
    m = re.match(r"v\[(\d+):(\d+)\]", spec)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", spec)
    return {int(m.group(1))} if m else set()


def _stage_loop(asm: str, kernel_re: str):
    """Instructions of the MFMA stage loop: the blocks of the depth-2 loop with the most MFMAs,
    in layout order rotated to start at the loop header (the compiler may place the latch block
    before the header)."""
    lines = asm.splitlines()
    start = next(i for i, l in enumerate(lines) if re.match(r"^_Z\S*" + kernel_re + r"\S*:", l))
    end = next(i for i in range(start + 1, len(lines))
               if re.match(r"^_Z\S+:", lines[i]) or "amdhsa.kernels" in lines[i])
    blocks, cur = [], None        # [name, header it belongs to (or None), lines]
    for line in lines[start:end]:
        m = re.match(r"^(\.LBB\d+_\d+):|^; (%bb\.\d+):", line)
        if m:
            h = re.search(r"Loop: Header=(BB\d+_\d+) Depth=2", line)
            cur = [re.sub(r"^\.L", "", m.group(1) or m.group(2)), h.group(1) if h else None, []]
            if "Loop Header: Depth=2" in line:
                cur[1] = cur[0]
            blocks.append(cur)
        elif cur is not None:
            if "Loop Header: Depth=2" in line:
                cur[1] = cur[0]
            cur[2].append(line)
    loops = {}
    for name, header, body in blocks:
        if header:
            loops.setdefault(header, []).append((name, body))
    header, best = max(loops.items(),
                       key=lambda hb: sum("v_mfma" in l for _, b in hb[1] for l in b))
    names = [n for n, _ in best]
    k = names.index(header) if header in names else 0
    order = best[k:] + best[:k]
    return [l for _, b in order for l in b]


def _read_to_use(loop):
    """MFMAs issued between each LDS read and the first MFMA that consumes its registers, over
    two passes of the loop (so reads consumed by the next iteration count too)."""
    pending, n, dists = [], 0, []
    for line in loop + loop:
        t = line.strip().split()
        if not t:
            continue
        if t[0].startswith("ds_read"):
            pending.append((_regs(t[1].rstrip(",")), n))
        elif t[0].startswith("v_mfma"):
            ops = [x.rstrip(",") for x in t[1:5]]
            used = _regs(ops[1]) | _regs(ops[2])
            for p in [p for p in pending if p[0] & used]:
                dists.append(n - p[1])
                pending.remove(p)
            n += 1
    return dists


@pytest.fixture(scope="module")
def asm(stats):
    return _assembly()


@pytest.mark.parametrize("bm,gateup", [(256, 1), (256, 0), (128, 1), (128, 0)])
def test_prefill_stage_loops_hide_lds_latency(asm, bm, gateup):
    loop = _stage_loop(asm, f"moe_tile_kernelILi{bm}ELb{gateup}")
    # 2 k-steps per stage x (FM x FN) fragments per wavefront: 8 x 4 at 256 rows, 4 x 4 at 128
    assert sum("v_mfma" in l for l in loop) == (64 if bm == 256 else 32)
    d = _read_to_use(loop)
    assert len(d) >= 24 and min(d) >= 6, sorted(d)
