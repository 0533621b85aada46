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


def _by_grid(path, counters=None):
    """{(kernel, grid): {counter: average}} from one --pmc CSV."""
    vals = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            if counters and r["Counter_Name"] not in counters:
                continue
            vals[(short_name(r["Kernel_Name"]), int(r["Grid_Size"]), r["Counter_Name"])].append(float(r["Counter_Value"]))
    out = collections.defaultdict(dict)
    for (k, g, c), v in vals.items():
        out[(k, g)][c] = sum(v) / len(v)
    return out


def step_table(db, fetch_csv, write_csv, mfma_csv, fetch_factor, write_factor, xcds=8, simds=1024,
               skip=("at::native", "__amd_rocclr", "weight_quant_kernel", "row_amax_kernel", "channel_scale_kernel")):
    con = sqlite3.connect(db)
    dur = collections.defaultdict(list)
    for name, gx, gy, gz, wx, start, end in con.execute(
            "select name, grid_x, grid_y, grid_z, workgroup_x, start, end from kernels"):
        k = short_name(name)
        if k.startswith(skip):
            continue
        dur[(k, gx * gy * gz)].append((end - start) / 1e3)
    fe, wr, mf = _by_grid(fetch_csv), _by_grid(write_csv), _by_grid(mfma_csv)
    steps = max(len(v) for k, v in dur.items() if k[0].startswith("readout_kernel")) if any(
        k[0].startswith("readout_kernel") for k in dur) else 1
    rows = []
    for (k, g), d in dur.items():
        us = sum(d) / len(d)
        byt = fe.get((k, g), {}).get("FETCH_SIZE", 0.0) * 1024 * fetch_factor + \
            wr.get((k, g), {}).get("WRITE_SIZE", 0.0) * 1024 * write_factor
        m = mf.get((k, g), {})
        busy = m.get("SQ_VALU_MFMA_BUSY_CYCLES")
        gui = m.get("GRBM_GUI_ACTIVE")
        util = 100.0 * busy / (gui / xcds * simds) if busy is not None and gui else None
        rows.append((k, g, len(d) / steps, us, sum(d) / steps, byt, byt / (us * 1e3) if us else 0.0, util))
    rows.sort(key=lambda r: -r[4])
    return rows


def format_step_table(rows, hbm_peak_gbs=8000.0):
    lines = [f"{'kernel':44s} {'threads':>8s} {'calls/step':>10s} {'avg_us':>8s} {'us/step':>9s} "
             f"{'MB/call':>8s} {'GB/s':>7s} {'%HBM':>6s} {'MFMA%':>6s}"]
    for k, g, calls, us, tot, byt, gbs, util in rows:
        lines.append(f"{k[:44]:44s} {g:8d} {calls:10.1f} {us:8.2f} {tot:9.1f} {byt / 1e6:8.2f} {gbs:7.0f} "
                     f"{100 * gbs / hbm_peak_gbs:6.1f} {'' if util is None else f'{util:6.1f}'}")
    lines.append(f"{'total':44s} {'':8s} {'':10s} {'':8s} {sum(r[4] for r in rows):9.1f}")
    return "\n".join(lines)


def main(argv):
    if len(argv) >= 2 and argv[0] == "kernels":
        print(format_kernel_stats(kernel_stats(argv[1])))
    elif len(argv) == 7 and argv[0] == "step":
        print(format_step_table(step_table(argv[1], argv[2], argv[3], argv[4], float(argv[5]), float(argv[6]))))
    elif len(argv) >= 2 and argv[0] == "pmc":
        for (k, c), (v, n) in sorted(pmc_averages(argv[1:]).items()):
            print(f"{k[:64]:64s} {c:14s} dispatches={n:4d} avg={v:.1f}")
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
