"""Summaries of rocprofv3 output for the committed profiles (no GPU needed).

    python -m tinyserve_amd.profiling stats <run_kernel_stats.csv> [--match SUBSTR ...]
        markdown table of per-kernel call count and average / total duration
    python -m tinyserve_amd.profiling traffic --fetch F.csv --write W.csv \
            --copy-fetch CF.csv --copy-write CW.csv --copy-bytes N --kernel SUBSTR
        HBM bytes per dispatch of one kernel from FETCH_SIZE / WRITE_SIZE counter collections,
        each scaled by the factor the same counter shows for a plain device copy of N bytes
    python -m tinyserve_amd.profiling counters <run_counter_collection.csv> ... [--match SUBSTR ...]
        markdown table of every counter's mean per dispatch, per kernel (e.g. MfmaUtil and
        SQ_INSTS_VALU_MFMA_MOPS_BF16 of the tile kernels), over one or more collections
"""
import argparse
import collections
import csv
import json
import re
import sys


def short_name(name: str) -> str:
    m = re.search(r"(\w+_kernel(?:<[^()]*>)?)", name)
    return m.group(1) if m else name[:80]


def kernel_stats(path):
    rows = list(csv.DictReader(open(path)))
    out = []
    for r in rows:
        out.append((r["Name"], int(r["Calls"]), float(r["AverageNs"]), float(r["TotalDurationNs"])))
    return out


def counter_per_kernel(path, counter):
    agg = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] == counter:
            agg[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in agg.items()}


def _pick(d, sub):
    hits = {k: v for k, v in d.items() if sub in k}
    if not hits:
        raise SystemExit(f"no kernel matching {sub!r}")
    return max(hits.items(), key=lambda kv: kv[1])


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--match", nargs="*", default=["tsm::"])
    t = sub.add_parser("traffic")
    for a in ("--fetch", "--write", "--copy-fetch", "--copy-write", "--kernel"):
        t.add_argument(a, required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--copy-kernel", default="copy")
    c = sub.add_parser("counters")
    c.add_argument("csv", nargs="+")
    c.add_argument("--match", nargs="*", default=["tsm::"])
    args = ap.parse_args(argv)

    if args.cmd == "counters":
        table = collections.defaultdict(dict)
        for path in args.csv:
            agg = collections.defaultdict(list)
            for r in csv.DictReader(open(path)):
                if any(m in r["Kernel_Name"] for m in args.match):
                    agg[(r["Kernel_Name"], r["Counter_Name"])].append(float(r["Counter_Value"]))
            for (k, name), v in agg.items():
                table[k][name] = sum(v) / len(v)
        names = sorted({n for row in table.values() for n in row})
        print("| kernel | " + " | ".join(names) + " |")
        print("|---|" + "---:|" * len(names))
        for k in sorted(table):
            cells = [f"{table[k][n]:.4g}" if n in table[k] else "" for n in names]
            print(f"| `{short_name(k)}` | " + " | ".join(cells) + " |")
        return 0

    if args.cmd == "stats":
        print("| kernel | calls | avg us | total us |")
        print("|---|---:|---:|---:|")
        for name, calls, avg, tot in kernel_stats(args.csv):
            if any(m in name for m in args.match):
                print(f"| `{short_name(name)}` | {calls} | {avg / 1e3:.2f} | {tot / 1e3:.1f} |")
        return 0

    f_k, f_kib = _pick(counter_per_kernel(args.fetch, "FETCH_SIZE"), args.kernel)
    w_k, w_kib = _pick(counter_per_kernel(args.write, "WRITE_SIZE"), args.kernel)
    _, cf_kib = _pick(counter_per_kernel(args.copy_fetch, "FETCH_SIZE"), args.copy_kernel)
    _, cw_kib = _pick(counter_per_kernel(args.copy_write, "WRITE_SIZE"), args.copy_kernel)
    f_factor = cf_kib * 1024 / args.copy_bytes   # counter bytes per byte actually read
    w_factor = cw_kib * 1024 / args.copy_bytes
    res = {
        "kernel": short_name(f_k),
        "fetch_kib": f_kib, "write_kib": w_kib,
        "copy_bytes": args.copy_bytes, "copy_fetch_kib": cf_kib, "copy_write_kib": cw_kib,
        "fetch_factor": f_factor, "write_factor": w_factor,
        "traffic_bytes": f_kib * 1024 / f_factor + w_kib * 1024 / w_factor,
    }
    json.dump(res, sys.stdout, indent=1)
    print()
    return 0


if __name__ == "__main__":
    sys.exit(main())
