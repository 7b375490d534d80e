"""Summarize rocprofv3 CSV output for this library's kernels.

    python -m aspida_amd.rocprof_summary TRACE_CSV [--pmc COUNTER_CSV ...] [--match REGEX]

TRACE_CSV is a ``*_kernel_trace.csv`` (``rocprofv3 --kernel-trace -f csv``):
dispatches are grouped by kernel symbol and grid, with count and mean /
median / min / max duration in microseconds.  Each COUNTER_CSV is a
``*_counter_collection.csv`` (``rocprofv3 --pmc ... -f csv``); its counters are
averaged per kernel symbol and grid.  Output is Markdown.
"""
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


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("trace")
    ap.add_argument("--pmc", nargs="*", default=[])
    ap.add_argument("--match", default=r"^kq_")
    args = ap.parse_args()
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
