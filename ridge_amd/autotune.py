"""Model-pruned empirical autotuner, evaluated offline on a measured sweep.

    python -m ridge_amd.autotune [--measured data/measured/mi355x.csv]
                                 [--hw data/hardware/mi355x.json] [--k 1,2,3,5,10,20]

Restates the reference's tools/ridge-autotune.py:41-129. The model ranks, the
hardware decides: per shape, the configs are sorted by predicted throughput
(a STABLE sort, so tied predictions keep table order), the top k are
"benchmarked" by looking up their measured throughput, and the regret is the
gap between the best of those k and the exhaustive best. Predictions come from
`ridge-predict --batch`; the model is never re-implemented here, and the
rounded (6 significant digit) strings it writes are what is ranked, ties
included.

Beside the model, the same regret is reported for rankings that need no model
(the comparison of the reference's README.md:81): a uniformly random shortlist
(its exact expected regret), the largest tile first (BM x BN, then BK), the
highest theoretical occupancy first and the highest arithmetic intensity first
(a plain roofline); the last two read the model's own occupancy and intensity
columns, with table order breaking ties.
"""

import argparse
import os
import statistics
import sys
import tempfile

from ridge_amd import model as RM
from ridge_amd import stats as S
from ridge_amd import tables as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEFAULT_KS = (1, 2, 3, 5, 10, 20)

# Rankings without a model: each maps a (measured record, predicted record) pair
# to a score, higher first.
HEURISTICS = {
    "largest tile": lambda m, p: (int(m["BM"]) * int(m["BN"]), int(m["BK"])),
    "occupancy": lambda m, p: float(p["pred_occ_factor"]),
    "roofline": lambda m, p: float(p["pred_arith_intensity"]),
}


def load_rows(path):
    return T.read(path).records


def predicted_rows(measured, hw, binary=None):
    with tempfile.TemporaryDirectory() as tmp:
        out = os.path.join(tmp, "pred.csv")
        RM.predict_batch(measured, out, hw=hw, binary=binary or RM.PREDICT_BIN)
        return T.read(out, require=("pred_tflops",)).records


def group_by_shape(meas, pred, score=None):
    """{tag: [(score, measured TFLOP/s), ...]} in table order. --batch preserves
    row order, so the join is positional; `score` defaults to the prediction."""
    if len(pred) != len(meas):
        raise ValueError("prediction/measurement row count mismatch: %d vs %d" % (len(pred), len(meas)))
    shapes = {}
    for m, p in zip(meas, pred):
        s = score(m, p) if score else float(p["pred_tflops"])
        shapes.setdefault(m["tag"], []).append((s, float(m["tflops"])))
    return shapes


def regret_at_k(shapes, k):
    """(mean regret %, max regret %, exact hits, per-shape regrets) at shortlist size k."""
    regrets, hits = [], 0
    for rows in shapes.values():
        best = max(r[1] for r in rows)
        shortlist = sorted(rows, key=lambda r: r[0], reverse=True)[:k]
        picked = max(r[1] for r in shortlist)
        regrets.append(S.regret(best, picked) * 100.0)
        hits += picked == best
    return statistics.mean(regrets), max(regrets), hits, regrets


def random_regret_at_k(shapes, k):
    """(mean, max) over shapes of the expected regret % of a random shortlist of k."""
    per = [S.expected_random_regret([r[1] for r in rows], k) * 100.0 for rows in shapes.values()]
    return statistics.mean(per), max(per)


def evaluate(measured, hw, ks=DEFAULT_KS, binary=None):
    meas = load_rows(measured)
    pred = predicted_rows(measured, hw, binary)
    shapes = group_by_shape(meas, pred)
    per_shape = len(meas) // len(shapes)
    table = []
    for k in ks:
        if k > per_shape:
            continue
        mean_r, max_r, hits, _ = regret_at_k(shapes, k)
        benches = k * len(shapes)
        table.append(dict(k=k, benchmarks=benches, reduction=len(meas) / benches, mean_regret=mean_r,
                          max_regret=max_r, hits=hits, shapes=len(shapes)))
    return table, len(meas), len(shapes), per_shape


def baselines(measured, hw, ks=DEFAULT_KS, binary=None):
    """{k: {name: (mean regret %, max regret %)}} for the random shortlist and
    the model-free rankings."""
    meas = load_rows(measured)
    pred = predicted_rows(measured, hw, binary)
    by_heuristic = {name: group_by_shape(meas, pred, f) for name, f in HEURISTICS.items()}
    shapes = group_by_shape(meas, pred)
    per_shape = min(len(v) for v in shapes.values())
    out = {}
    for k in ks:
        if k > per_shape:
            continue
        row = {"random": random_regret_at_k(shapes, k)}
        for name, grouped in by_heuristic.items():
            mean_r, max_r, _, _ = regret_at_k(grouped, k)
            row[name] = (mean_r, max_r)
        out[k] = row
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--measured", default=os.path.join(ROOT, "data", "measured", "mi355x.csv"))
    ap.add_argument("--hw", default=os.path.join(ROOT, "data", "hardware", "mi355x.json"))
    ap.add_argument("--predict-bin", default=RM.PREDICT_BIN, help="the ridge-predict executable")
    ap.add_argument("--k", default=",".join(str(k) for k in DEFAULT_KS),
                    help="shortlist sizes to evaluate, per shape")
    ap.add_argument("--target-k", type=int, default=10)
    ap.add_argument("--target-regret", type=float, default=2.0)
    args = ap.parse_args(argv)
    if not os.path.exists(args.measured):
        sys.exit("missing %s" % args.measured)
    hw = args.hw if (args.hw in ("a100", "mi355x") or os.path.exists(args.hw)) else "mi355x"
    ks = [int(x) for x in args.k.split(",")]
    try:
        table, total, nshapes, per_shape = evaluate(args.measured, hw, ks, args.predict_bin)
        base = baselines(args.measured, hw, ks, args.predict_bin)
    except (T.TableError, RuntimeError) as e:
        sys.exit(str(e))

    print("Model-pruned empirical autotuner")
    print("  measured sweep   %s" % args.measured)
    print("  hardware model   %s" % hw)
    print("  %d configs over %d shapes (%d per shape)" % (total, nshapes, per_shape))
    print()
    print("  %5s %12s %13s %11s %11s %10s" % ("top_k", "benchmarks", "vs exhaustive", "mean regret",
                                               "max regret", "exact hits"))
    best_k = None
    for row in table:
        print("  %5d %12d %12.1fx %10.2f%% %10.2f%% %6d/%-3d" % (
            row["k"], row["benchmarks"], row["reduction"], row["mean_regret"], row["max_regret"], row["hits"],
            row["shapes"]))
        if best_k is None and row["mean_regret"] <= 3.0:
            best_k = row
    print()
    names = ["random"] + list(HEURISTICS)
    print("  mean (max) regret of rankings without the model:")
    print("  %5s %s" % ("top_k", "".join("%22s" % n for n in names)))
    for k in sorted(base):
        print("  %5d %s" % (k, "".join("%22s" % ("%.2f%% (%.1f%%)" % base[k][n]) for n in names)))
    print()
    if best_k:
        print("  Smallest k within 3%% of exhaustive: k=%d (%d benchmarks instead of %d, %.1fx fewer)"
              % (best_k["k"], best_k["benchmarks"], total, best_k["reduction"]))
    else:
        print("  No k reached within 3% of exhaustive: the ranking is not strong enough to prune this space.")
    target = [r for r in table if r["k"] == args.target_k]
    if target:
        ok = target[0]["mean_regret"] <= args.target_regret
        print("  target: mean regret <= %.1f%% at k=%d -> %.2f%% %s" % (
            args.target_regret, args.target_k, target[0]["mean_regret"], "MET" if ok else "NOT MET"))
        return 0 if ok else 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
