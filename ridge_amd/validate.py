"""Joins a measured sweep with model predictions and reports accuracy and ranking
separately: a model can be good at one and bad at the other.

    python -m ridge_amd.validate [--measured data/measured/mi355x.csv]
                                 [--registered data/sweep/mi355x-registered.csv]
                                 [--hw data/hardware/mi355x.json]

Restates the reference's bench/validate.py:36-359: MAPE with its distribution,
tie-averaged Spearman per shape, rank-of-best and regret@1 as [pessimistic,
optimistic] ranges over predicted ties, the predicted label distribution, and
the gate that the measured set is exactly the registered cross product of
shapes x kernel table. The kernel table comes from the C ABI
(ridge_gemm_variant_table_csv) instead of a regex over a source file. Statistics
are written out, not imported; predictions come from `ridge-predict --batch`.
Exit code 1 when a gate fails (MAPE ceiling, cross-product mismatch).
"""

import argparse
import collections
import csv
import os
import sys
import tempfile

from ridge_amd import model as RM

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def average_ranks(xs):
    """1-based ranks with ties averaged (what Spearman requires)."""
    order = sorted(range(len(xs)), key=lambda i: xs[i])
    ranks = [0.0] * len(xs)
    i = 0
    while i < len(order):
        j = i
        while j + 1 < len(order) and xs[order[j + 1]] == xs[order[i]]:
            j += 1
        avg = (i + j) / 2.0 + 1.0
        for k in range(i, j + 1):
            ranks[order[k]] = avg
        i = j + 1
    return ranks


def pearson(a, b):
    n = len(a)
    if n < 2:
        return float("nan")
    ma, mb = sum(a) / n, sum(b) / n
    num = sum((x - ma) * (y - mb) for x, y in zip(a, b))
    da = sum((x - ma) ** 2 for x in a) ** 0.5
    db = sum((y - mb) ** 2 for y in b) ** 0.5
    if da == 0.0 or db == 0.0:
        return float("nan")  # no variance on one side: a result, not an accident
    return num / (da * db)


def spearman(a, b):
    return pearson(average_ranks(a), average_ranks(b))


def percentile(xs, p):
    if not xs:
        return float("nan")
    s = sorted(xs)
    if len(s) == 1:
        return s[0]
    idx = (len(s) - 1) * p / 100.0
    lo, hi = int(idx), min(int(idx) + 1, len(s) - 1)
    return s[lo] + (s[hi] - s[lo]) * (idx - lo)


def rank_bounds(rows, key_pred="pred_tflops", key_meas="tflops"):
    """(best, worst) rank of the measured-best config in the predicted order."""
    best = max(rows, key=lambda r: float(r[key_meas]))
    p = float(best[key_pred])
    better = sum(1 for r in rows if float(r[key_pred]) > p)
    tied = sum(1 for r in rows if float(r[key_pred]) == p)
    return better + 1, better + tied


def regret_bounds(rows, key_pred="pred_tflops", key_meas="tflops"):
    """(worst, best, tie size) fraction lost by taking the predicted top pick."""
    measured_best = max(float(r[key_meas]) for r in rows)
    top = max(float(r[key_pred]) for r in rows)
    tied = [float(r[key_meas]) for r in rows if float(r[key_pred]) == top]
    return (measured_best - min(tied)) / measured_best, (measured_best - max(tied)) / measured_best, len(tied)


def load_registered(path):
    shapes = []
    for line in open(path):
        line = line.strip()
        if not line or line.startswith("#"):
            continue
        p = line.split(",")
        shapes.append((int(p[0]), int(p[1]), int(p[2])))
    return shapes


def load_variant_table():
    from ridge_amd import gemm as G
    rows = list(csv.DictReader(G.variant_table_csv().splitlines()))
    return [tuple(int(r[k]) for k in ("BM", "BN", "BK", "WM", "WN", "stages", "groupM")) for r in rows]


def cross_product_gate(rows, registered, variants):
    expected = {(M, N, K) + v for (M, N, K) in registered for v in variants}
    got = {tuple(int(r[k]) for k in ("M", "N", "K", "BM", "BN", "BK", "WM", "WN", "stages", "groupM"))
           for r in rows}
    return expected - got, got - expected


def read_meta(path):
    meta = {}
    for line in open(path):
        if line.startswith("#"):
            parts = line[1:].strip().split(",", 1)
            if len(parts) == 2:
                meta[parts[0].strip()] = parts[1].strip()
    return meta


SCHEDULE_NAMES = {"0": "uniform", "1": "ping-pong", "2": "persistent"}


def error_by_resident_waves(rows, simds_per_cu=4):
    """MAPE and mean signed error per (resident wavefronts per SIMD, schedule)
    class: workgroups resident per CU (the model's ctasPerSM) x wavefronts per
    workgroup / SIMDs per CU. Needs the pred_ctas_per_sm column and a per-row
    schedule; returns {} for CSVs without them (the reference's A100 sweep)."""
    if not rows or "pred_ctas_per_sm" not in rows[0] or "schedule" not in rows[0]:
        return {}
    acc = {}
    for r in rows:
        waves = (int(r["BM"]) // int(r["WM"])) * (int(r["BN"]) // int(r["WN"]))
        per_simd = int(float(r["pred_ctas_per_sm"])) * waves / simds_per_cu
        key = (per_simd, "%d-wave %s" % (waves, SCHEDULE_NAMES.get(r["schedule"], r["schedule"])))
        n, a, sg = acc.get(key, (0, 0.0, 0.0))
        acc[key] = (n + 1, a + r["_abs"], sg + r["_signed"])
    return {k: (n, a / n, sg / n) for k, (n, a, sg) in acc.items()}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--measured", default=os.path.join(ROOT, "data", "measured", "mi355x.csv"))
    ap.add_argument("--registered", default=os.path.join(ROOT, "data", "sweep", "mi355x-registered.csv"))
    ap.add_argument("--hw", default=os.path.join(ROOT, "data", "hardware", "mi355x.json"))
    ap.add_argument("--max-mape", type=float, default=10.0)
    ap.add_argument("--fail-mape", type=float, default=15.0)
    ap.add_argument("--no-table-gate", action="store_true",
                    help="skip the cross-product gate (e.g. for another GPU's sweep)")
    args = ap.parse_args(argv)
    for p in (args.measured, args.registered):
        if not os.path.exists(p):
            sys.exit("missing %s" % p)

    meta = read_meta(args.measured)
    print("=" * 74)
    print("ridge model validation")
    print("=" * 74)
    for k in ("gpu", "cus", "sms", "nominal_clock_mhz", "warmup_seconds", "canary_drift_fraction"):
        if k in meta:
            print("  %-24s %s" % (k, meta[k]))
    print("  %-24s %s" % ("hardware model", args.hw))
    print()

    failures = []
    with tempfile.TemporaryDirectory() as td:
        pred_path = os.path.join(td, "pred.csv")
        sys.stderr.write(RM.predict_batch(args.measured, pred_path, hw=args.hw))
        rows = list(csv.DictReader(r for r in open(pred_path) if not r.startswith("#")))
    if not rows:
        sys.exit("no rows after prediction")

    if not args.no_table_gate:
        registered = load_registered(args.registered)
        variants = load_variant_table()
        missing, extra = cross_product_gate(rows, registered, variants)
        print("registered cross product: %d shapes x %d variants = %d" % (
            len(registered), len(variants), len(registered) * len(variants)))
        print("measured rows:            %d" % len(rows))
        if missing or extra:
            print("  MISSING from measured: %d, EXTRA in measured: %d" % (len(missing), len(extra)))
            for m in sorted(missing)[:5]:
                print("    %s" % (m,))
            failures.append("measured set does not match the registered sweep")
        else:
            print("  matches the registered sweep exactly")
        print()

    errs, signed = [], []
    for r in rows:
        m, p = float(r["tflops"]), float(r["pred_tflops"])
        r["_abs"] = abs(p - m) / m * 100.0
        r["_signed"] = (p - m) / m * 100.0
        errs.append(r["_abs"])
        signed.append(r["_signed"])
    mape = sum(errs) / len(errs)
    print("absolute accuracy")
    print("  %-22s %8.2f %%   (gate: <= %.0f%%)" % ("MAPE", mape, args.max_mape))
    print("  %-22s %8.2f %%" % ("median abs error", percentile(errs, 50)))
    print("  %-22s %8.2f %%" % ("p90 abs error", percentile(errs, 90)))
    print("  %-22s %8.2f %%" % ("max abs error", max(errs)))
    print("  %-22s %+8.2f %%   (negative = model under-predicts)" % ("mean signed error", sum(signed) / len(signed)))
    print()
    print("  worst 8 configs by absolute error:")
    print("    %-22s %-22s %9s %9s %8s" % ("shape", "tile/wave tile/stages", "measured", "predicted", "err%"))
    for r in sorted(rows, key=lambda r: -r["_abs"])[:8]:
        cfg = "%sx%sx%s w%sx%s s%s" % (r["BM"], r["BN"], r["BK"], r["WM"], r["WN"], r["stages"])
        print("    %-22s %-22s %9.1f %9.1f %+8.1f" % ("%sx%sx%s" % (r["M"], r["N"], r["K"]), cfg,
                                                    float(r["tflops"]), float(r["pred_tflops"]), r["_signed"]))
    print()
    classes = error_by_resident_waves(rows)
    if classes:
        # The wavefront analogue of the reference's 4-active-warp error class
        # (42 of its 336 A100 rows over-predicted by 39%, README.md:160).
        print("  by resident wavefronts per SIMD and schedule:")
        print("    %-11s %-20s %5s %8s %9s" % ("waves/SIMD", "workgroup", "rows", "MAPE %", "signed %"))
        for (w, sched), (n, a, sg) in sorted(classes.items()):
            print("    %-11s %-20s %5d %8.1f %+9.1f" % ("%g" % w, sched, n, a, sg))
        print()
    if mape > args.fail_mape:
        failures.append("MAPE %.1f%% is above the %.0f%% ceiling" % (mape, args.fail_mape))
    elif mape > args.max_mape:
        print("  note: MAPE %.1f%% exceeds the %.0f%% target (ranking quality is what the pruner uses)\n"
              % (mape, args.max_mape))

    by_shape = collections.OrderedDict()
    for r in rows:
        by_shape.setdefault((r["M"], r["N"], r["K"], r.get("tag", "")), []).append(r)
    print("ranking quality, per problem shape")
    print("  %-26s %8s %5s %13s %9s %14s" % ("shape", "spearman", "ties", "rank of best", "recall@3",
                                             "regret@1 %"))
    rhos, worst_regrets, ties = [], [], []
    for (M, N, K, tag), rs in by_shape.items():
        meas = [float(r["tflops"]) for r in rs]
        pred = [float(r["pred_tflops"]) for r in rs]
        rho = spearman(meas, pred)
        b, w = rank_bounds(rs)
        wr, br, nt = regret_bounds(rs)
        largest = max(collections.Counter(round(p, 6) for p in pred).values())
        rhos.append(rho)
        worst_regrets.append(wr)
        ties.append(largest)
        print("  %-26s %8s %5d %13s %9s %14s" % (
            (tag or "%sx%sx%s" % (M, N, K))[:26], "  n/a" if rho != rho else "%.3f" % rho, largest,
            "%d" % b if b == w else "%d-%d" % (b, w), "yes" if w <= 3 else ("maybe" if b <= 3 else "no"),
            "%.1f-%.1f" % (wr * 100, br * 100) if nt > 1 else "%.1f" % (wr * 100)))
    valid = [r for r in rhos if r == r]
    print()
    print("  %-26s %7.3f   (%d shapes without prediction variance)" % (
        "mean Spearman", sum(valid) / len(valid) if valid else float("nan"), len(rhos) - len(valid)))
    print("  %-26s %7.2f %%" % ("worst-case regret@1", max(worst_regrets) * 100))
    print("  %-26s %7d configs" % ("largest tie group", max(ties)))
    print()
    labels = collections.Counter(r["pred_bottleneck"] for r in rows)
    print("bottleneck attribution")
    print("  predicted label distribution: %s" % dict(labels))
    print("  counter cross-check: python -m ridge_amd.labelcheck (registered in data/sweep/rocprof-label-mapping.md)")
    print()
    print("=" * 74)
    print("MAPE %.2f%%, mean Spearman %.3f, worst regret@1 %.2f%%" % (
        mape, sum(valid) / len(valid) if valid else float("nan"), max(worst_regrets) * 100))
    if failures:
        for f in failures:
            print("  %s" % f)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
