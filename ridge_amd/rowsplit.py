"""Launch plans over the kernel table, ranked by the cost model.

    python -m ridge_amd.rowsplit rank --shape M,N,K [--hw data/hardware/mi355x.json] [--top 10]
    python -m ridge_amd.rowsplit register --sweeps a.csv,b.csv --measured x.csv,y.csv --out plans.csv
                                          [--hw ...] [--splits 5]
    python -m ridge_amd.rowsplit score --plans plans.csv --measured plans-measured.csv [--hw ...]

A plan is one table row launched over the whole shape, or a row split: a body
row on the first rows of C, as many as make whole rounds of its resident
workgroups (ridge_gemm_split_rows), and a tail row on the rest, two launches on
one stream (ridge_gemm_launch_split). The model ranks plans by predicted time; a
split's is the two launches' predicted times added (each launch's prediction
already carries the launch boundary when the calibration switches launchModel
on). No counterpart in the reference, whose autotuner (tools/ridge-autotune.py)
ranks single kernel-table rows only.

`register` writes the plans a measurement of the split decision times, per shape
of the given registered sweeps that has at least one split: the row measured
fastest on it in the given sweep CSVs (the anchor), the model's best single row,
and the model's best `--splits` split plans with distinct (body rows, tail row)
pairs, each with its best-predicted body row (body rows of one tile family
predict within a fraction of a percent of each other, so the plain top five
would time five bodies with one tail). `ridge-measure --plans` times them
(the `register` output is its input). `score` reports, per shape, the best
measured split against the best measured single row, and the regret of the
model's first choice with and without splits among its candidates.
"""

import argparse
import os
import statistics
import sys
from collections import namedtuple

from ridge_amd import gemm as G
from ridge_amd import model as RM
from ridge_amd import tables as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KEY = ("BM", "BN", "BK", "WM", "WN", "stages", "groupM")
PLAN_COLUMNS = (["M", "N", "K", "tag"] + list(KEY) + ["body_rows"] + ["tail_" + c for c in KEY]
                + ["role", "predicted_us"])
WHOLE_DEVICE_CUS = 256


class Plan(namedtuple("Plan", "M N K body rows tail seconds")):
    """`body`, `tail`: kernel-table indices (tail None for one launch); `rows`: the
    body's rows of C (M for one launch); `seconds`: the model's time."""

    @property
    def split(self):
        return self.tail is not None

    def key(self):
        """(body key, body rows, tail key) as the plan CSVs hold it."""
        b = G.variant(self.body).key()
        t = G.variant(self.tail).key() if self.split else (0,) * 7
        return (self.M, self.N, self.K) + b + (self.rows,) + t

    def label(self):
        body = G.variant(self.body).label()
        if not self.split:
            return body
        return "%s on %d rows + %s on %d" % (body, self.rows, G.variant(self.tail).label(), self.M - self.rows)


class Ranker:
    """The model's time for every (row, sub-shape) it is asked, computed once."""

    def __init__(self, hw_path, num_cus=WHOLE_DEVICE_CUS):
        self.hw = RM.Hardware(hw_path)
        self.num_cus = num_cus
        self.rows = G.variants()
        self._seconds = {}

    def seconds(self, i, M, N, K):
        key = (i, M, N, K)
        if key not in self._seconds:
            v = self.rows[i]
            p = RM.predict(self.hw, M=M, N=N, K=K, BM=v.BM, BN=v.BN, BK=v.BK, warpM=v.WM, warpN=v.WN,
                           stages=v.stages, regsPerThread=v.regsPerThread, groupM=v.groupM, schedule=v.schedule)
            self._seconds[key] = 2.0 * M * N * K / (p["predictedTFLOPS"] * 1e12)
        return self._seconds[key]

    def singles(self, M, N, K):
        return [Plan(M, N, K, v.index, M, None, self.seconds(v.index, M, N, K))
                for v in self.rows if v.divides(M, N, K)]

    def splits(self, M, N, K):
        out = []
        for b in self.rows:
            rows = G.split_rows(b.index, M, N, K, self.num_cus)
            if not 0 < rows < M:
                continue
            body = self.seconds(b.index, rows, N, K)
            for t in self.rows:
                if t.divides(M - rows, N, K):
                    out.append(Plan(M, N, K, b.index, rows, t.index, body + self.seconds(t.index, M - rows, N, K)))
        return out

    def rank(self, M, N, K):
        """Every single row and split plan of the shape, fastest predicted first;
        ties keep table order, singles before splits."""
        return sorted(self.singles(M, N, K) + self.splits(M, N, K), key=lambda p: p.seconds)


def _measured_best(paths):
    """{(M, N, K): kernel-table index of the row measured fastest} over sweep CSVs."""
    best = {}
    for path in paths:
        for r in T.read(path, require=("M", "N", "K", "tflops") + KEY).records:
            s = (int(r["M"]), int(r["N"]), int(r["K"]))
            tf = float(r["tflops"])
            if s not in best or tf > best[s][0]:
                best[s] = (tf, G.find_variant(*(int(r[c]) for c in KEY)))
    return {s: i for s, (tf, i) in best.items()}


def _record(plan, tag, role):
    body = G.variant(plan.body).key()
    tail = G.variant(plan.tail).key() if plan.split else (0,) * 7
    r = {"M": plan.M, "N": plan.N, "K": plan.K, "tag": tag, "body_rows": plan.rows, "role": role,
         "predicted_us": "%.3f" % (plan.seconds * 1e6)}
    r.update(zip(KEY, body))
    r.update(zip(("tail_" + c for c in KEY), tail))
    return r


def distinct_splits(ranker, M, N, K, n):
    """The model's best `n` split plans with distinct (body rows, tail row) pairs,
    fastest predicted first; within a pair, the best-predicted body row (table
    order on ties)."""
    best = {}
    for p in sorted(ranker.splits(M, N, K), key=lambda p: p.seconds):
        best.setdefault((p.rows, p.tail), p)
    return sorted(best.values(), key=lambda p: p.seconds)[:n]


def register(shapes, measured_paths, ranker, n_splits=5):
    """The plan records for every shape with at least one split: the anchor (the
    measured-fastest row), the model's best single row when it is another, and
    the model's best `n_splits` distinct splits. Shapes with no split are left
    out."""
    anchors = _measured_best(measured_paths)
    out = []
    for (M, N, K, tag) in shapes:
        splits = distinct_splits(ranker, M, N, K, n_splits)
        if not splits:
            continue
        if (M, N, K) not in anchors or anchors[(M, N, K)] < 0:
            raise ValueError("no measured row for %dx%dx%d in the sweep CSVs" % (M, N, K))
        anchor = anchors[(M, N, K)]
        out.append(_record(Plan(M, N, K, anchor, M, None, ranker.seconds(anchor, M, N, K)), tag, "anchor"))
        top = min(ranker.singles(M, N, K), key=lambda p: p.seconds)
        if top.body != anchor:
            out.append(_record(top, tag, "model_single"))
        for j, p in enumerate(splits, start=1):
            out.append(_record(p, tag, "model_split_%d" % j))
    return out


def _plan_key(r):
    return tuple(int(r[c]) for c in ["M", "N", "K"] + list(KEY) + ["body_rows"] + ["tail_" + c for c in KEY])


def score(plans_path, measured_path, ranker):
    """Per shape of the measured plans: the best measured single row and split,
    the split's gain, the measured outcome of the model's first choice over
    singles only and over singles and splits (its regret against the best
    measured plan), and the best plan against hipBLASLt. Every registered plan
    must have been measured."""
    registered = T.read(plans_path, require=PLAN_COLUMNS).records
    measured = {}
    for r in T.read(measured_path, require=("tflops", "blas_tflops")).records:
        measured[_plan_key(r)] = r
    missing = [r for r in registered if _plan_key(r) not in measured]
    if missing:
        raise ValueError("%d registered plans were not measured (first: %s)"
                         % (len(missing), ",".join(str(x) for x in _plan_key(missing[0]))))
    shapes = {}
    for r in registered:
        shapes.setdefault((int(r["M"]), int(r["N"]), int(r["K"]), r["tag"]), []).append(r)
    rows = []
    for (M, N, K, tag), recs in shapes.items():
        tf = {_plan_key(r): float(measured[_plan_key(r)]["tflops"]) for r in recs}
        singles = [k for r, k in ((r, _plan_key(r)) for r in recs) if int(r["body_rows"]) == M]
        splits = [k for r, k in ((r, _plan_key(r)) for r in recs) if int(r["body_rows"]) != M]
        best_single = max(tf[k] for k in singles)
        best_split = max(tf[k] for k in splits)
        best = max(best_single, best_split)
        ranked = ranker.rank(M, N, K)
        first_any = ranked[0].key()
        first_single = next(p for p in ranked if not p.split).key()
        for k in (first_any, first_single):
            if k not in tf:
                raise ValueError("the model's first choice %s on %dx%dx%d was not registered" % (k, M, N, K))
        blas = statistics.median(float(measured[k]["blas_tflops"]) for k in tf)
        rows.append({"M": M, "N": N, "K": K, "tag": tag, "best_single": best_single, "best_split": best_split,
                     "gain": best_split / best_single, "model_picks_split": ranked[0].split,
                     "regret_singles": (best - tf[first_single]) / best * 100,
                     "regret_with_splits": (best - tf[first_any]) / best * 100,
                     "blas": blas, "best_vs_blas": best / blas, "best_single_vs_blas": best_single / blas})
    return rows


def _print_rank(ranker, M, N, K, top):
    plans = ranker.rank(M, N, K)
    print("%dx%dx%d: %d single rows, %d split plans" % (M, N, K, sum(not p.split for p in plans),
                                                         sum(p.split for p in plans)))
    for p in plans[:top]:
        print("  %9.1f TFLOP/s  %8.2f us  %s" % (2.0 * M * N * K / p.seconds / 1e12, p.seconds * 1e6, p.label()))


def _print_score(rows):
    print("%-22s %9s %9s %7s %6s %9s %9s %7s" % ("shape", "single", "split", "gain", "pick", "reg.1row", "reg.plan",
                                                "x blas"))
    for r in rows:
        print("%-22s %9.1f %9.1f %6.3fx %6s %8.2f%% %8.2f%% %6.3fx" % (
            "%dx%dx%d" % (r["M"], r["N"], r["K"]), r["best_single"], r["best_split"], r["gain"],
            "split" if r["model_picks_split"] else "row", r["regret_singles"], r["regret_with_splits"],
            r["best_vs_blas"]))
    n = len(rows)
    gains = [r["gain"] for r in rows]
    print("\n%d shapes; the best split beats the best single row by more than 1%% on %d, by more than 5%% on %d; "
          "median gain %.3fx, highest %.3fx" % (n, sum(g > 1.01 for g in gains), sum(g > 1.05 for g in gains),
                                               statistics.median(gains), max(gains)))
    for name in ("regret_singles", "regret_with_splits"):
        xs = [r[name] for r in rows]
        print("model's first choice, %s: mean regret %.2f%%, worst %.2f%%"
              % ("single rows only" if name == "regret_singles" else "rows and splits", statistics.mean(xs), max(xs)))
    print("model picks a split on %d shapes; faster than hipBLASLt with the best plan on %d of %d "
          "(best single row: %d)" % (sum(r["model_picks_split"] for r in rows), sum(r["best_vs_blas"] > 1 for r in rows),
                                     n, sum(r["best_single_vs_blas"] > 1 for r in rows)))


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    hw_default = os.path.join(ROOT, "data", "hardware", "mi355x.json")
    r = sub.add_parser("rank")
    r.add_argument("--shape", required=True)
    r.add_argument("--hw", default=hw_default)
    r.add_argument("--top", type=int, default=10)
    g = sub.add_parser("register")
    g.add_argument("--sweeps", required=True, help="registered shape lists, comma-separated")
    g.add_argument("--measured", required=True, help="measured sweep CSVs for the anchors, comma-separated")
    g.add_argument("--out", required=True)
    g.add_argument("--hw", default=hw_default)
    g.add_argument("--splits", type=int, default=5)
    s = sub.add_parser("score")
    s.add_argument("--plans", required=True)
    s.add_argument("--measured", required=True)
    s.add_argument("--hw", default=hw_default)
    args = ap.parse_args(argv)
    ranker = Ranker(args.hw)
    if args.cmd == "rank":
        M, N, K = (int(x) for x in args.shape.split(","))
        _print_rank(ranker, M, N, K, args.top)
    elif args.cmd == "register":
        shapes, seen = [], set()
        for path in args.sweeps.split(","):
            for s in T.read_shapes(path):
                if s[:3] not in seen:
                    seen.add(s[:3])
                    shapes.append(s)
        recs = register(shapes, args.measured.split(","), ranker, args.splits)
        comments = ["launch plans registered by python -m ridge_amd.rowsplit register (%d plans, %d shapes)"
                    % (len(recs), len({(r["M"], r["N"], r["K"]) for r in recs})),
                    "hw,%s" % os.path.relpath(args.hw, ROOT)]
        T.write(args.out, PLAN_COLUMNS, recs, comments)
        print("%s: %d plans" % (args.out, len(recs)))
    else:
        _print_score(score(args.plans, args.measured, ranker))
    return 0


if __name__ == "__main__":
    sys.exit(main())
