"""Summarize rocprofv3 CSV output for this library's kernels.

    python -m aspida_amd.rocprof_summary TRACE_CSV [--pmc COUNTER_CSV ...] [--match REGEX]
        [--traffic FETCH_CSV WRITE_CSV --probe-kib N --traffic-json OUT]

TRACE_CSV is a ``*_kernel_trace.csv`` (``rocprofv3 --kernel-trace -f csv``):
dispatches are grouped by kernel symbol and grid, with count and mean /
median / min / max duration in microseconds.  Each COUNTER_CSV is a
``*_counter_collection.csv`` (``rocprofv3 --pmc ... -f csv``); its counters are
averaged per kernel symbol and grid.  Output is Markdown.

With --traffic, the FETCH_SIZE and WRITE_SIZE runs (KiB per dispatch) are
turned into HBM bytes per launch of each kernel symbol: each counter is scaled
by what it reads for the probe copy (the __amd_rocclr_copyBuffer dispatch of
N KiB read and N KiB written in the same run), and the per-symbol means are
written to OUT as JSON {"kernels": {symbol: {"traffic_bytes_per_launch": ...}}}.
"""
import json
import argparse
import collections
import csv
import re
import statistics


def short_name(name):
    """'void kq::kq_mv_packed<0, 16>(unsigned char const*, ...)' -> 'kq_mv_packed<0, 16>'."""
    head = name.split("(")[0]
    head = re.sub(r"^void\s+", "", head)
    return head.split("::")[-1] if "::" in head else head


def _col(row, *names):
    for n in names:
        if n in row:
            return row[n]
    raise KeyError(names)


def trace_groups(path, match):
    groups = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            name = short_name(r["Kernel_Name"])
            if not re.search(match, name):
                continue
            grid = f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}/{r['Workgroup_Size_X']}"
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
            groups[(name, grid)].append(us)
    return groups


def counter_groups(path, match):
    groups = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            name = short_name(r["Kernel_Name"])
            if not re.search(match, name):
                continue
            grid = _col(r, "Grid_Size", "Grid_Size_X")
            wg = _col(r, "Workgroup_Size", "Workgroup_Size_X")
            groups[(name, f"{grid}/{wg}", r["Counter_Name"])].append(float(r["Counter_Value"]))
    return groups


def _symbol_means(path, counter, match):
    """(symbol -> (mean counter value per dispatch, dispatches), largest value of a copyBuffer dispatch)."""
    vals = collections.defaultdict(list)
    probe = None
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            name = short_name(r["Kernel_Name"])
            v = float(r["Counter_Value"])
            if "copyBuffer" in name:
                probe = v if probe is None else max(probe, v)
            elif re.search(match, name):
                vals[name].append(v)
    return {k: (statistics.fmean(v), len(v)) for k, v in vals.items()}, probe


def traffic(fetch_csv, write_csv, probe_kib, match):
    fetch, pf = _symbol_means(fetch_csv, "FETCH_SIZE", match)
    write, pw = _symbol_means(write_csv, "WRITE_SIZE", match)
    if pf is None or pw is None:
        raise SystemExit("no copy-probe dispatch in the counter runs (bench.py --copy-probe-mib)")
    # The probe is the largest copy dispatch of each run.
    fs, ws = probe_kib / pf, probe_kib / pw
    out = {"fetch_scale": round(fs, 6), "write_scale": round(ws, 6),
           "calibration": f"copy probe of {probe_kib} KiB: FETCH_SIZE {pf:.1f} KiB, WRITE_SIZE {pw:.1f} KiB",
           "kernels": {}}
    for k in sorted(set(fetch) & set(write)):
        b = (fetch[k][0] * fs + write[k][0] * ws) * 1024.0
        out["kernels"][k] = {"traffic_bytes_per_launch": int(round(b)), "dispatches": fetch[k][1],
                             "fetch_kib": round(fetch[k][0], 1), "write_kib": round(write[k][0], 1)}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("trace")
    ap.add_argument("--pmc", nargs="*", default=[])
    ap.add_argument("--match", default=r"^kq_")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--probe-kib", type=float, default=262144.0)
    ap.add_argument("--traffic-json")
    args = ap.parse_args()
    if args.traffic:
        t = traffic(args.traffic[0], args.traffic[1], args.probe_kib, args.match)
        if args.traffic_json:
            with open(args.traffic_json, "w") as f:
                json.dump(t, f, indent=1)
        print(f"Traffic per launch ({t['calibration']}; scales {t['fetch_scale']}, {t['write_scale']}):")
        print()
        print("| kernel | dispatches | FETCH KiB | WRITE KiB | HBM bytes per launch |")
        print("|---|---|---|---|---|")
        for k, v in t["kernels"].items():
            print(f"| {k} | {v['dispatches']} | {v['fetch_kib']} | {v['write_kib']} | {v['traffic_bytes_per_launch']} |")
        print()
    print("| kernel | grid/workgroup | dispatches | mean us | median us | min us | max us |")
    print("|---|---|---|---|---|---|---|")
    for (name, grid), v in sorted(trace_groups(args.trace, args.match).items()):
        print(f"| {name} | {grid} | {len(v)} | {statistics.fmean(v):.2f} | {statistics.median(v):.2f} | "
              f"{min(v):.2f} | {max(v):.2f} |")
    for path in args.pmc:
        print()
        print(f"Counters from {path.split('/')[-1]} (mean per dispatch):")
        print()
        print("| kernel | grid/workgroup | counter | dispatches | mean |")
        print("|---|---|---|---|---|")
        for (name, grid, ctr), v in sorted(counter_groups(path, args.match).items()):
            print(f"| {name} | {grid} | {ctr} | {len(v)} | {statistics.fmean(v):.1f} |")


if __name__ == "__main__":
    main()
