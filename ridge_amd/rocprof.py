"""Readers for rocprofv3 CSV output, and a per-phase summary of one profiled run.

    python -m ridge_amd.rocprof phases --trace D [--counters D ...] [--min-run N]

A run of `bench.py` launches the same kernel in long contiguous stretches: the
clock ramp and the timed windows, hipBLASLt's windows, the fills of the cold
operand sets, the cold rotation. `phases` splits the dispatches, in dispatch
order, into maximal runs of one kernel name and prints, for every run of at least
N dispatches, the duration statistics (kernel trace) and the per-dispatch median
of every collected counter (counter collection). Counters of one dispatch that
rocprofv3 reports per XCD or per instance are summed, except the GRBM_* clock
counts, which count the same cycles on every XCD: for those the per-XCD value is
taken (the largest instance, or the sum over the XCDs divided by their number when
reported summed).

The traffic counters are raw: FETCH_SIZE and WRITE_SIZE are in KiB per dispatch
and are scaled by what the same counter reads for a device copy of known size
(`bench.py --mode copy`; on gfx950 FETCH_SIZE reads half the copy's bytes and
WRITE_SIZE all of them, hence the factors 2 and 1 below).
"""

import argparse
import csv
import glob
import os
import statistics
import sys

FETCH_SCALE = 2.000
WRITE_SCALE = 1.000
XCDS = 8


def find(directory, suffix):
    hits = sorted(glob.glob(os.path.join(directory, "**", "*" + suffix), recursive=True))
    if not hits:
        raise SystemExit("no *%s under %s" % (suffix, directory))
    return hits


def parse_counter_dir(directory):
    """{(file, dispatch_id): {"name": kernel, "counters": {name: [values]}}} for
    every dispatch of every *counter_collection.csv under `directory`."""
    out = {}
    for path in find(directory, "counter_collection.csv"):
        with open(path) as f:
            for r in csv.DictReader(f):
                d = out.setdefault((path, int(r["Dispatch_Id"])), {"name": r["Kernel_Name"], "counters": {}})
                d["counters"].setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return out


def parse_trace_dir(directory):
    """{(file, dispatch_id): {"name": kernel, "ns": duration}} for every dispatch
    of every *kernel_trace.csv under `directory`."""
    out = {}
    for path in find(directory, "kernel_trace.csv"):
        with open(path) as f:
            for r in csv.DictReader(f):
                out[(path, int(r["Dispatch_Id"]))] = {
                    "name": r["Kernel_Name"], "ns": float(r["End_Timestamp"]) - float(r["Start_Timestamp"])}
    return out


def counter_value(dispatch, name, xcds=XCDS):
    vals = dispatch["counters"].get(name)
    if vals is None:
        raise SystemExit("counter %s missing from a dispatch" % name)
    if name.startswith("GRBM_"):
        return max(vals) if len(vals) > 1 else vals[0] / xcds
    return sum(vals)


def short_name(name):
    """The kernel's function name without its template arguments or parameters,
    mangled or demangled."""
    s = name
    if s.startswith("_Z"):
        i = 2
        if s[i] == "N":  # nested name: take the last component
            i += 1
        parts = []
        while i < len(s) and s[i].isdigit():
            j = i
            while j < len(s) and s[j].isdigit():
                j += 1
            n = int(s[i:j])
            if j + n > len(s):
                break
            parts.append(s[j:j + n])
            i = j + n
        if parts:
            return parts[-1]
    for sep in ("<", "("):
        if sep in s:
            s = s[:s.index(sep)]
    # A demangled name may carry its return type ("void ns::kernel").
    words = s.split("::")[-1].split()
    return words[-1] if words else name


def phases(parsed, min_run=1):
    """Maximal runs of one kernel name in dispatch order, as (name, [dispatch])
    pairs, keeping runs of at least `min_run` dispatches."""
    runs = []
    for _, d in sorted(parsed.items()):
        if runs and runs[-1][0] == d["name"]:
            runs[-1][1].append(d)
        else:
            runs.append((d["name"], [d]))
    return [(n, ds) for n, ds in runs if len(ds) >= min_run]


def _pct(xs, q):
    ys = sorted(xs)
    return ys[min(len(ys) - 1, int(q * (len(ys) - 1) + 0.5))]


def trace_table(parsed, min_run):
    rows = []
    for i, (name, ds) in enumerate(phases(parsed, min_run)):
        us = [d["ns"] * 1e-3 for d in ds]
        rows.append({"phase": i, "kernel": short_name(name), "launches": len(us),
                     "median_us": statistics.median(us), "p10_us": _pct(us, 0.10), "p90_us": _pct(us, 0.90),
                     "mean_us": statistics.fmean(us)})
    return rows


def counter_table(parsed, min_run):
    rows = []
    for i, (name, ds) in enumerate(phases(parsed, min_run)):
        names = sorted(ds[0]["counters"])
        row = {"phase": i, "kernel": short_name(name), "launches": len(ds)}
        for c in names:
            row[c] = statistics.median(counter_value(d, c) for d in ds)
        if "FETCH_SIZE" in row:
            row["fetch_bytes"] = row["FETCH_SIZE"] * FETCH_SCALE * 1024.0
        if "WRITE_SIZE" in row:
            row["write_bytes"] = row["WRITE_SIZE"] * WRITE_SCALE * 1024.0
        rows.append(row)
    return rows


def _print_rows(rows):
    if not rows:
        print("(no phase)")
        return
    cols = []
    for r in rows:
        cols += [k for k in r if k not in cols]
    print("| " + " | ".join(cols) + " |")
    print("|" + "---|" * len(cols))
    for r in rows:
        cells = []
        for k in cols:
            v = r.get(k, "")
            cells.append("%.6g" % v if isinstance(v, float) else str(v))
        print("| " + " | ".join(cells) + " |")


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    p = sub.add_parser("phases")
    p.add_argument("--trace", default=None, help="rocprofv3 output directory of a --kernel-trace run")
    p.add_argument("--counters", action="append", default=[], help="rocprofv3 output directory of a --pmc run")
    p.add_argument("--min-run", type=int, default=1, help="drop runs of fewer dispatches")
    args = ap.parse_args(argv)
    if args.trace:
        print("## kernel trace: %s" % args.trace)
        _print_rows(trace_table(parse_trace_dir(args.trace), args.min_run))
    for d in args.counters:
        print("\n## counters: %s" % d)
        _print_rows(counter_table(parse_counter_dir(d), args.min_run))
    return 0


if __name__ == "__main__":
    sys.exit(main() or 0)
