"""The rocprofv3 summary tool on synthetic CSVs (no GPU): kernel-name shortening, the stats table,
and the traffic arithmetic (each counter divided by what it reads for a copy of known size)."""
import csv
import io
import json
from contextlib import redirect_stdout

from tinyserve_amd import profiling

K = "void tsm::(anonymous namespace)::moe_expert_kernel<16, 2, 1, true, true, 1>(tsm::ExpertArgs)"
COPY = "void at::native::elementwise_kernel<128, 4>(int, copy_kernel_functor)"


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def _counters(path, counter, kernel, values):
    _write(path, ["Kernel_Name", "Counter_Name", "Counter_Value"],
           [[kernel, counter, v] for v in values])


def test_short_name():
    assert profiling.short_name(K) == "moe_expert_kernel<16, 2, 1, true, true, 1>"


def test_stats_table(tmp_path):
    p = tmp_path / "stats.csv"
    _write(p, ["Name", "Calls", "AverageNs", "TotalDurationNs"],
           [[K, 4, 130000.0, 520000.0], ["other_kernel", 1, 5.0, 5.0]])
    buf = io.StringIO()
    with redirect_stdout(buf):
        profiling.main(["stats", str(p)])
    lines = buf.getvalue().splitlines()
    assert lines[2] == "| `moe_expert_kernel<16, 2, 1, true, true, 1>` | 4 | 130.00 | 520.0 |"
    assert len(lines) == 3  # only kernels of this package


def test_traffic(tmp_path):
    copy_bytes = 1 << 30
    _counters(tmp_path / "f.csv", "FETCH_SIZE", K, [1000.0, 1200.0])      # mean 1100 KiB
    _counters(tmp_path / "w.csv", "WRITE_SIZE", K, [10.0])
    _counters(tmp_path / "cf.csv", "FETCH_SIZE", COPY, [copy_bytes / 1024 / 2])  # reads half
    _counters(tmp_path / "cw.csv", "WRITE_SIZE", COPY, [copy_bytes / 1024])
    buf = io.StringIO()
    with redirect_stdout(buf):
        profiling.main(["traffic", "--fetch", str(tmp_path / "f.csv"),
                        "--write", str(tmp_path / "w.csv"),
                        "--copy-fetch", str(tmp_path / "cf.csv"),
                        "--copy-write", str(tmp_path / "cw.csv"),
                        "--copy-bytes", str(copy_bytes), "--kernel", "moe_expert_kernel"])
    res = json.loads(buf.getvalue())
    assert res["fetch_factor"] == 0.5 and res["write_factor"] == 1.0
    assert res["traffic_bytes"] == 1100 * 1024 / 0.5 + 10 * 1024


def test_counters_table(tmp_path):
    _counters(tmp_path / "a.csv", "MfmaUtil", K, [30.0, 34.0])
    _write(tmp_path / "b.csv", ["Kernel_Name", "Counter_Name", "Counter_Value"],
           [[K, "SQ_INSTS_VALU_MFMA_MOPS_BF16", 8.0], [COPY, "MfmaUtil", 1.0]])
    buf = io.StringIO()
    with redirect_stdout(buf):
        profiling.main(["counters", str(tmp_path / "a.csv"), str(tmp_path / "b.csv")])
    lines = buf.getvalue().splitlines()
    assert lines[0] == "| kernel | MfmaUtil | SQ_INSTS_VALU_MFMA_MOPS_BF16 |"
    assert lines[2] == "| `moe_expert_kernel<16, 2, 1, true, true, 1>` | 32 | 8 |"
    assert len(lines) == 3  # the copy kernel is not this package's
