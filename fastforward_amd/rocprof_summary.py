"""Summaries of rocprofv3 output for the kernels of this library.

``python -m fastforward_amd.rocprof_summary kernels <results.db>`` prints per
kernel name the dispatch count, total and average duration and share of the
total (``--kernel-trace`` rocpd database). ``python -m
fastforward_amd.rocprof_summary pmc <counter_collection.csv> [...]`` prints the
average counter value per dispatch for every kernel name and counter found in
``--pmc`` CSV output.
"""
import collections
import csv
import re
import sqlite3
import sys


def short_name(name):
    name = name.replace("(anonymous namespace)::", "")
    name = re.sub(r"\(.*", "", name)
    return re.sub(r"^void ", "", name).strip()


def kernel_stats(db):
    con = sqlite3.connect(db)
    cur = con.cursor()
    cols = [r[1] for r in cur.execute("pragma table_info(kernels)")]
    name_col = "kernel_name" if "kernel_name" in cols else "name"
    agg = collections.OrderedDict()
    for name, start, end in cur.execute(f"select {name_col}, start, end from kernels"):
        a = agg.setdefault(short_name(name), [0, 0.0])
        a[0] += 1
        a[1] += (end - start) / 1e3
    return agg


def format_kernel_stats(agg):
    tot = sum(v[1] for v in agg.values()) or 1.0
    lines = [f"{'kernel':64s} {'calls':>6s} {'total_us':>10s} {'avg_us':>9s} {'pct':>6s}"]
    for k, (n, t) in sorted(agg.items(), key=lambda x: -x[1][1]):
        lines.append(f"{k[:64]:64s} {n:6d} {t:10.1f} {t / n:9.2f} {100 * t / tot:6.2f}")
    lines.append(f"total_us {tot:.1f}")
    return "\n".join(lines)


def pmc_averages(paths):
    """{(kernel, counter): average value per dispatch} over rocprofv3 --pmc CSV files."""
    vals = collections.defaultdict(list)
    for path in paths:
        with open(path) as f:
            for r in csv.DictReader(f):
                vals[(short_name(r["Kernel_Name"]), r["Counter_Name"])].append(float(r["Counter_Value"]))
    return {k: (sum(v) / len(v), len(v)) for k, v in vals.items()}


def main(argv):
    if len(argv) >= 2 and argv[0] == "kernels":
        print(format_kernel_stats(kernel_stats(argv[1])))
    elif len(argv) >= 2 and argv[0] == "pmc":
        for (k, c), (v, n) in sorted(pmc_averages(argv[1:]).items()):
            print(f"{k[:64]:64s} {c:14s} dispatches={n:4d} avg={v:.1f}")
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
