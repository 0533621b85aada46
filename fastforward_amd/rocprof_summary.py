"""Summaries of rocprofv3 output for the kernels of this library.

``python -m fastforward_amd.rocprof_summary kernels <results.db>`` prints per
kernel name the dispatch count, total and average duration and share of the
total (``--kernel-trace`` rocpd database). ``python -m
fastforward_amd.rocprof_summary pmc <counter_collection.csv> [...]`` prints the
average counter value per dispatch for every kernel name and counter found in
``--pmc`` CSV output. ``python -m fastforward_amd.rocprof_summary steptrace
<results.db>`` prints per-step kernel time (model-construction kernels left
out; a step is one readout launch) and ``step <results.db> <fetch.csv>
<write.csv> <mfma.csv> <fetch_factor> <write_factor>`` adds bytes per call and
MFMA busy % from the three counter runs. ``traffic <fetch.csv> <write.csv>
<manifest.json>`` turns the two counter runs of ``bench.py --kernels`` (and the
launch manifest that command prints) into HBM bytes per GEMM launch, scaled by
what the counters read for its 256 MiB calibration copy, and writes the JSON
summary to stdout after the table.
"""
import json
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
               skip=("at::native", "__amd_rocclr", "weight_quant_kernel", "row_amax_kernel", "channel_scale_kernel",
                     "int4_quant_kernel", "pack_fp8_kernel", "pack_int4_kernel", "pack_scales_int4_kernel",
                     "pack_bf16_kernel", "tensor_scale_kernel")):
    con = sqlite3.connect(db)
    dur = collections.defaultdict(list)
    for name, gx, gy, gz, wx, start, end in con.execute(
            "select name, grid_x, grid_y, grid_z, workgroup_x, start, end from kernels"):
        k = short_name(name)
        if k.startswith(skip):
            continue
        dur[(k, gx * gy * gz)].append((end - start) / 1e3)
    fe, wr, mf = (_by_grid(p) if p else {} for p in (fetch_csv, write_csv, mfma_csv))
    steps = 1  # a step is one readout launch (LM step) or one pixel packing launch (vision step)
    for first in ("readout_kernel", "pack_pixels_kernel"):
        if any(k[0].startswith(first) for k in dur):
            steps = max(len(v) for k, v in dur.items() if k[0].startswith(first))
            break
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


def format_step_table(rows, hbm_peak_gbs=8000.0, counters=True):
    if not counters:
        lines = [f"{'kernel':44s} {'threads':>8s} {'calls/step':>10s} {'avg_us':>8s} {'us/step':>9s}"]
        for k, g, calls, us, tot, *_ in rows:
            lines.append(f"{k[:44]:44s} {g:8d} {calls:10.1f} {us:8.2f} {tot:9.1f}")
        lines.append(f"{'total':44s} {'':8s} {'':10s} {'':8s} {sum(r[4] for r in rows):9.1f}")
        return "\n".join(lines)
    lines = [f"{'kernel':44s} {'threads':>8s} {'calls/step':>10s} {'avg_us':>8s} {'us/step':>9s} "
             f"{'MB/call':>8s} {'GB/s':>7s} {'%HBM':>6s} {'MFMA%':>6s}"]
    for k, g, calls, us, tot, byt, gbs, util in rows:
        lines.append(f"{k[:44]:44s} {g:8d} {calls:10.1f} {us:8.2f} {tot:9.1f} {byt / 1e6:8.2f} {gbs:7.0f} "
                     f"{100 * gbs / hbm_peak_gbs:6.1f} {'' if util is None else f'{util:6.1f}'}")
    lines.append(f"{'total':44s} {'':8s} {'':10s} {'':8s} {sum(r[4] for r in rows):9.1f}")
    return "\n".join(lines)


def _dispatches(path):
    """[(dispatch id, kernel, {counter: value})] in dispatch order from one --pmc CSV."""
    rows = collections.OrderedDict()
    with open(path) as f:
        for r in csv.DictReader(f):
            d = rows.setdefault(int(r["Dispatch_Id"]), [short_name(r["Kernel_Name"]), {}])
            d[1][r["Counter_Name"]] = d[1].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [(i, k, c) for i, (k, c) in sorted(rows.items())]


def _launches(dispatches):
    """GEMM launches from dispatches in order: a gemm_fp8*/gemv_fp8* dispatch plus
    the split_reduce_kernel dispatch that follows it for a k-split launch, counters
    summed, kernel names joined with '+'."""
    out = []
    for i, k, c in dispatches:
        if k.startswith(("gemm_fp8", "gemv_fp8")):
            out.append((i, k, dict(c)))
        elif k.startswith("split_reduce_kernel") and out:
            j, k0, c0 = out[-1]
            out[-1] = (j, f"{k0} + {k}", {n: c0.get(n, 0.0) + v for n, v in c.items()})
    return out


def traffic(fetch_csv, write_csv, manifest):
    """GEMM launches of ``bench.py --kernels`` in manifest order (``reps`` each),
    then the calibration copy (the last ``copy_reps`` dispatches)."""
    fe, wr = _dispatches(fetch_csv), _dispatches(write_csv)
    reps = manifest["copy_reps"]
    f_copy = sum(c["FETCH_SIZE"] for _, _, c in fe[-reps:]) / reps
    w_copy = sum(c["WRITE_SIZE"] for _, _, c in wr[-reps:]) / reps
    ff = manifest["copy_bytes"] / (f_copy * 1024)
    wf = manifest["copy_bytes"] / (w_copy * 1024)
    gf, gw = _launches(fe[:-reps]), _launches(wr[:-reps])
    out, pos, tot_b, tot_n = [], 0, 0.0, 0
    for e in manifest["gemm_launches"]:
        n = e["reps"]
        fk = sum(c["FETCH_SIZE"] for _, _, c in gf[pos:pos + n]) / n
        wk = sum(c["WRITE_SIZE"] for _, _, c in gw[pos:pos + n]) / n
        kern = gf[pos][1]
        pos += n
        hbm = fk * 1024 * ff + wk * 1024 * wf
        out.append(dict(shape=e["shape"], kernel=kern, launches_per_step=e["launches_per_step"],
                        fetch_kib=round(fk, 1), write_kib=round(wk, 1), hbm_bytes=int(hbm),
                        algorithmic_bytes=e["algorithmic_bytes"], ratio=round(hbm / e["algorithmic_bytes"], 2)))
        tot_b += hbm * e["launches_per_step"]
        tot_n += e["launches_per_step"]
    return dict(kernel="FP8 GEMM launches of the step (per shape below)", bytes_per_launch=int(tot_b / tot_n),
                launches_per_step=tot_n,
                calibration=dict(copy_bytes=manifest["copy_bytes"], fetch_kib=round(f_copy, 1),
                                 write_kib=round(w_copy, 1), fetch_factor=round(ff, 4), write_factor=round(wf, 4)),
                by_shape=out)


def format_traffic(t):
    lines = ["| shape (M x K x N) | kernel | launches/step | FETCH KiB | WRITE KiB | HBM bytes | algorithmic bytes | ratio |",
             "|---|---|---|---|---|---|---|---|"]
    for r in t["by_shape"]:
        lines.append(f"| {r['shape']} | `{r['kernel']}` | {r['launches_per_step']} | {r['fetch_kib']} | "
                     f"{r['write_kib']} | {r['hbm_bytes'] / 1e6:.1f} MB | {r['algorithmic_bytes'] / 1e6:.1f} MB | "
                     f"{r['ratio']} |")
    lines.append(f"\nStep-weighted bytes per launch: {t['bytes_per_launch'] / 1e6:.1f} MB "
                 f"({t['launches_per_step']} launches per step); calibration factors FETCH "
                 f"{t['calibration']['fetch_factor']}, WRITE {t['calibration']['write_factor']}.")
    return "\n".join(lines)


def main(argv):
    if len(argv) >= 2 and argv[0] == "kernels":
        print(format_kernel_stats(kernel_stats(argv[1])))
    elif len(argv) == 4 and argv[0] == "traffic":
        with open(argv[3]) as f:
            man = json.loads([ln for ln in f if ln.startswith("{")][-1])
        t = traffic(argv[1], argv[2], man)
        print(format_traffic(t))
        print(json.dumps(t, indent=1))
    elif len(argv) == 2 and argv[0] == "steptrace":
        print(format_step_table(step_table(argv[1], None, None, None, 1.0, 1.0), counters=False))
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
