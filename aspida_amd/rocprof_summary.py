"""Summarize rocprofv3 CSV output for this library's kernels.

    python -m aspida_amd.rocprof_summary TRACE_CSV [--pmc COUNTER_CSV ...] [--match REGEX]
        [--traffic FETCH_CSV WRITE_CSV --probe-kib N --traffic-json OUT]

TRACE_CSV is a ``*_kernel_trace.csv`` (``rocprofv3 --kernel-trace -f csv``):
dispatches are grouped by kernel symbol and grid, with count and mean /
median / min / max duration in microseconds.  Each COUNTER_CSV is a
``*_counter_collection.csv`` (``rocprofv3 --pmc ... -f csv``); its counters are
averaged per kernel symbol and grid.  Output is Markdown.

--segment REGEX N splits the dispatches of every kernel whose symbol matches
REGEX into N consecutive parts (labelled #1..#N, in dispatch order) -- e.g.
a table that runs the same kernels at several sizes one after another.

--bench-rows small|kquant|sweep (with --traffic) prints one line per row of that
bench.py table instead: the run's dispatches are cut into rows at each random-
number kernel (every row draws its input first), a row's dispatches into its
1 + R ncopy products (bench.py's eager call and R graph replays of ncopy
weight copies), and each product's kernels get their median duration and
calibrated HBM bytes beside the row's algorithmic bytes.  With --pmc COUNTER_CSV
instead of --traffic: each row's median duration and its counters' means per
dispatch, with the VALU and MFMA busy shares they imply.

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


def _unmangle(name):
    """'_ZN2kq9kq_xsplitILi32EEEvPKf...' -> 'kq_xsplit<32>': the last name of an
    Itanium nested name and its integer / bool template arguments (the profiler
    leaves names mangled when it cannot demangle a parameter type, _Float16)."""
    i, ident = 3, None
    while i < len(name) and name[i].isdigit():
        j = i
        while name[j].isdigit():
            j += 1
        n = int(name[i:j])
        ident, i = name[j:j + n], j + n
    if ident is None:
        return name
    args = []
    if i < len(name) and name[i] == "I":
        for m in re.finditer(r"L([ib])(n?\d+)E", name[i + 1:name.find("EE", i) + 1]):
            v = m.group(2).replace("n", "-")
            args.append(("true" if v == "1" else "false") if m.group(1) == "b" else v)
    return ident + (f"<{', '.join(args)}>" if args else "")


def short_name(name):
    """'void kq::kq_mv_packed<0, 16>(unsigned char const*, ...)' -> 'kq_mv_packed<0, 16>'
    ('(anonymous namespace)::' scopes dropped first); mangled names by _unmangle."""
    if name.startswith("_ZN"):
        return _unmangle(name)
    head = name.replace("(anonymous namespace)::", "").split("(")[0]
    head = re.sub(r"^void\s+", "", head)
    return head.split("::")[-1] if "::" in head else head


def _col(row, *names):
    for n in names:
        if n in row:
            return row[n]
    raise KeyError(names)


SEGMENTS = []  # (regex, parts) from --segment


def _segmented(groups):
    """Split each group whose symbol matches a --segment regex into its parts."""
    out = {}
    for key, vals in groups.items():
        parts = next((n for rx, n in SEGMENTS if re.search(rx, key[0])), 1)
        if parts > 1 and len(vals) % parts == 0:
            m = len(vals) // parts
            for i in range(parts):
                out[(f"{key[0]} #{i + 1}",) + tuple(key[1:])] = vals[i * m:(i + 1) * m]
        else:
            out[key] = vals
    return out


def trace_groups(path, match):
    groups = collections.defaultdict(list)
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            name = short_name(r["Kernel_Name"])
            if not re.search(match, name):
                continue
            rows.append((int(r["Start_Timestamp"]), name, r))
    for _, name, r in sorted(rows, key=lambda t: t[0]):
        grid = f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}/{r['Workgroup_Size_X']}"
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        groups[(name, grid)].append(us)
    return _segmented(groups)


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
    return _segmented(groups)


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
                vals[(name,)].append(v)
    return {k[0]: (statistics.fmean(v), len(v)) for k, v in _segmented(vals).items()}, probe


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


# The rows of bench.py's small_batch_table and kquant_table, in run order:
# (kind name, out_dim, in_dim, batch).
_KQ = ("Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K")
BENCH_ROWS = {
    "small": [(k, o, i, b) for k in ("Q4_K", "Q6_K") for o, i in ((4096, 4096), (14336, 4096))
              for b in (2, 4, 8, 16, 32, 64)],
    "kquant": [(k, o, i, 1) for k in _KQ for o, i in ((14336, 4096), (4096, 14336))] + [("Q4_K", 4096, 4096, 1)],
    # bench.py SWEEP_SHAPES per kind
    "sweep": [(k, o, i, 1) for k in _KQ for o, i in ((2048, 4096), (4096, 4096), (8192, 4096), (14336, 4096),
                                                      (28672, 4096), (57344, 4096), (57344, 8192))],
}
# Graph replays of each row (one untimed, then the timed ones).
BENCH_REPLAYS = {"small": 4, "kquant": 5, "sweep": 5}
# Busy-share reference for --bench-rows with --pmc: MI355X's 1024 SIMDs at its
# 2400 MHz peak engine clock.  A SIMD's vector ALU is 16 lanes wide, so a
# wave64 VALU instruction occupies it for 4 cycles (VALU_CYCLES); matrix-core
# instructions are counted in SQ_INSTS_VALU too and are taken out of it.
SIMDS, CLOCK_MHZ, VALU_CYCLES = 1024, 2400, 4
_BLOCK = {"Q4_K": 144, "Q6_K": 210, "Q5_K": 176, "Q3_K": 110, "Q2_K": 84}


def _row_dispatches(path, counter=None):
    """The library's dispatches (kq_*, but not the packing) of each table row,
    rows cut at every random-number kernel; rows with none are dropped."""
    recs = []
    with open(path) as f:
        for r in csv.DictReader(f):
            if counter is not None and r["Counter_Name"] != counter:
                continue
            recs.append(r)
    order = "Dispatch_Id" if counter is not None else "Start_Timestamp"
    recs.sort(key=lambda r: int(r[order]))
    rows, cur = [], None
    for r in recs:
        if "distribution" in r["Kernel_Name"]:
            cur = []
            rows.append(cur)
            continue
        name = short_name(r["Kernel_Name"])
        if cur is None or not name.startswith("kq_") or name.startswith("kq_pack"):
            continue
        v = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0 if counter is None else \
            float(r["Counter_Value"])
        cur.append((name, v))
    return [r for r in rows if r]


def bench_rows(table, trace_csv, fetch_csv, write_csv, probe_kib):
    t = traffic(fetch_csv, write_csv, probe_kib, r"^kq_")
    fs, ws = t["fetch_scale"], t["write_scale"]
    tr, fe, wr = _row_dispatches(trace_csv), _row_dispatches(fetch_csv, "FETCH_SIZE"), \
        _row_dispatches(write_csv, "WRITE_SIZE")
    spec = BENCH_ROWS[table]
    if not len(tr) == len(fe) == len(wr) == len(spec):
        raise SystemExit(f"rows found: trace {len(tr)}, fetch {len(fe)}, write {len(wr)}; expected {len(spec)}")
    print(f"Per row ({t['calibration']}; scales {fs}, {ws}); duration = sum of the product's kernels' "
          "median durations; algorithmic bytes = weights + 4 B (in + out):")
    print()
    print("| row | kernels of one product, median µs each | µs | algorithmic bytes | GB/s | HBM bytes "
          "per product | HBM / weights |")
    print("|---|---|---|---|---|---|---|")
    for (kind, o, i, b), rt, rf, rw in zip(spec, tr, fe, wr):
        wbytes = _BLOCK[kind] * o * (i // 256)
        ncopy = max(8, -(-int(1.1 * (1 << 30)) // wbytes))
        calls = 1 + BENCH_REPLAYS[table] * ncopy
        k = len(rt) // calls
        if k * calls != len(rt) or len(rf) != len(rt) or len(rw) != len(rt):
            raise SystemExit(f"{kind} {o}x{i} B={b}: {len(rt)} dispatches for {calls} products")
        names = [rt[j][0] for j in range(k)]
        med = [statistics.median(rt[c * k + j][1] for c in range(1, calls)) for j in range(k)]
        hbm = 1024 * sum(statistics.fmean(rf[c * k + j][1] for c in range(1, calls)) * fs +
                         statistics.fmean(rw[c * k + j][1] for c in range(1, calls)) * ws for j in range(k))
        alg = wbytes + 4 * b * (i + o)
        us = sum(med)
        label = f"{kind} {o}x{i}" + (f" B={b}" if table == "small" else "")
        print(f"| {label} | {' + '.join(f'{n} {m:.2f}' for n, m in zip(names, med))} | {us:.2f} | {alg} | "
              f"{alg / us / 1e3:.0f} | {int(hbm)} | {hbm / wbytes:.3f} |")


def bench_rows_pmc(table, trace_csv, pmc_csv):
    """Per row: the median duration of its kernel (trace run) and the mean
    per dispatch of every counter of the counter run; VALU busy =
    (SQ_INSTS_VALU - SQ_INSTS_MFMA) x VALU_CYCLES / (SIMDS x duration x
    CLOCK_MHZ), MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDS x duration x
    CLOCK_MHZ)."""
    with open(pmc_csv) as f:
        names = sorted({r["Counter_Name"] for r in csv.DictReader(f)})
    tr = _row_dispatches(trace_csv)
    pm = {n: _row_dispatches(pmc_csv, n) for n in names}
    spec = BENCH_ROWS[table]
    if len(tr) != len(spec) or any(len(v) != len(spec) for v in pm.values()):
        raise SystemExit(f"rows found: trace {len(tr)}, counters {[len(v) for v in pm.values()]}; expected {len(spec)}")
    print(f"Per row: median duration (trace run), counters as the mean per dispatch (counter run); VALU busy "
          f"({VALU_CYCLES} cycles per non-MFMA VALU instruction) and MFMA busy against {SIMDS} SIMDs at {CLOCK_MHZ} MHz "
          f"for the traced duration:")
    print()
    print("| row | kernel | µs | GB/s | " + " | ".join(names) + " | VALU busy | MFMA busy |")
    print("|---|---|---|---|" + "---|" * len(names) + "---|---|")
    for r, (kind, o, i, b) in enumerate(spec):
        label = f"{kind} {o}x{i}" + (f" B={b}" if table == "small" else "")
        nbytes = _BLOCK[kind] * o * (i // 256) + 4 * b * (i + o)
        # one line per kernel of the row (a pre-pass and its product apart)
        for kn in dict.fromkeys(n for n, _ in tr[r]):
            us = statistics.median(v for n, v in tr[r] if n == kn)
            mean = {c: statistics.fmean(v for n, v in pm[c][r] if n == kn) for c in names}
            cyc = SIMDS * us * CLOCK_MHZ
            valu = (mean.get("SQ_INSTS_VALU", 0.0) - mean.get("SQ_INSTS_MFMA", 0.0)) * VALU_CYCLES / cyc
            mfma = mean.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / cyc
            print(f"| {label} | {kn} | {us:.2f} | {nbytes / us / 1e3:.0f} | " +
                  " | ".join(f"{mean[c]:.0f}" for c in names) + f" | {valu:.2f} | {mfma:.2f} |")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("trace")
    ap.add_argument("--pmc", nargs="*", default=[])
    ap.add_argument("--match", default=r"^kq_")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--probe-kib", type=float, default=262144.0)
    ap.add_argument("--traffic-json")
    ap.add_argument("--segment", nargs=2, action="append", default=[], metavar=("REGEX", "N"))
    ap.add_argument("--bench-rows", choices=sorted(BENCH_ROWS))
    args = ap.parse_args()
    SEGMENTS.extend((rx, int(n)) for rx, n in args.segment)
    if args.bench_rows and args.pmc and not args.traffic:
        bench_rows_pmc(args.bench_rows, args.trace, args.pmc[0])
        return
    if args.bench_rows:
        if not args.traffic:
            raise SystemExit("--bench-rows needs --traffic or --pmc")
        bench_rows(args.bench_rows, args.trace, args.traffic[0], args.traffic[1], args.probe_kib)
        return
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
