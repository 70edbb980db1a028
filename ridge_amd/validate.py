"""Accuracy report: the model's predictions against a measured sweep.

    python -m ridge_amd.validate [--measured data/measured/mi355x.csv]
                                 [--registered data/sweep/mi355x-registered.csv]
                                 [--hw data/hardware/mi355x.json]

Counterpart of the reference's bench/validate.py:36-359, with the same report
contents: absolute error (MAPE, median, p90, max, mean signed error), ranking
quality per shape (Spearman's rho on mid-ranks, the predicted position of the
measured-best config and the regret of the predicted top pick, both as ranges
over predicted ties, since a tie is not a decision the model made), the
predicted label distribution, and the integrity gate that the measured rows are
exactly the registered shapes x the kernel table. Here the table is read from
the C ABI (ridge_gemm_variant_table_csv), and the report adds the error by
resident wavefronts per SIMD and schedule. Predictions come from
`ridge-predict --batch`; statistics are in ridge_amd.stats, tables are read by
ridge_amd.tables. Exit code 1 when a gate fails.
"""

import argparse
import collections
import math
import os
import sys
import tempfile
from dataclasses import dataclass

from ridge_amd import model as RM
from ridge_amd import stats as S
from ridge_amd import tables as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KEY_COLUMNS = ("BM", "BN", "BK", "WM", "WN", "stages", "groupM")
SCHEDULES = {"0": "uniform", "1": "ping-pong", "2": "persistent"}


def kernel_table_keys():
    """The 7-field key of every row of the built kernel table, in table order."""
    from ridge_amd import gemm as G
    table = T.parse(G.variant_table_csv().splitlines(), "ridge_gemm_variant_table_csv()", require=KEY_COLUMNS)
    return [tuple(table.number(i, c, int) for c in KEY_COLUMNS) for i in range(len(table))]


def registered_gate(records, shapes, keys):
    """(absent, unexpected): registered (shape + key) rows that were not measured,
    and measured rows that were not registered."""
    want = {(M, N, K) + key for (M, N, K, _tag) in shapes for key in keys}
    have = {tuple(int(r[c]) for c in ("M", "N", "K") + KEY_COLUMNS) for r in records}
    return want - have, have - want


@dataclass
class Joined:
    """One measured row with the model's prediction for it."""
    record: dict
    measured: float
    predicted: float

    @property
    def signed_pct(self):
        return (self.predicted - self.measured) / self.measured * 100.0

    @property
    def abs_pct(self):
        return abs(self.signed_pct)


def join(measured_path, hw, binary=None):
    with tempfile.TemporaryDirectory() as td:
        out = os.path.join(td, "pred.csv")
        sys.stderr.write(RM.predict_batch(measured_path, out, hw=hw, binary=binary or RM.PREDICT_BIN))
        table = T.read(out, require=("M", "N", "K", "tflops", "pred_tflops", "pred_bottleneck") + KEY_COLUMNS)
    return [Joined(r, table.number(i, "tflops"), table.number(i, "pred_tflops")) for i, r in enumerate(table)]


def error_by_resident_waves(rows, simds_per_cu=4):
    """{(waves per SIMD, workgroup kind): (rows, MAPE %, mean signed %)}. A row's
    resident wavefronts per SIMD are its predicted workgroups per CU times its
    wavefronts per workgroup over the SIMDs of a CU. Empty for tables without
    the pred_ctas_per_sm and schedule columns (the reference's A100 sweep)."""
    if not rows or not {"pred_ctas_per_sm", "schedule"} <= set(rows[0].record):
        return {}
    groups = collections.defaultdict(list)
    for j in rows:
        r = j.record
        waves = (int(r["BM"]) // int(r["WM"])) * (int(r["BN"]) // int(r["WN"]))
        per_simd = int(float(r["pred_ctas_per_sm"])) * waves / simds_per_cu
        kind = "%d-wave %s" % (waves, SCHEDULES.get(r["schedule"], r["schedule"]))
        groups[(per_simd, kind)].append(j)
    return {key: (len(js), sum(j.abs_pct for j in js) / len(js), sum(j.signed_pct for j in js) / len(js))
            for key, js in groups.items()}


@dataclass
class ShapeRanking:
    tag: str
    rho: float
    largest_tie: int
    best_rank: tuple       # (optimistic, pessimistic)
    regret1: tuple         # (pessimistic, optimistic), fractions
    top_tie: int


def rank_shapes(rows):
    """One ShapeRanking per shape, in first-seen order."""
    shapes = collections.OrderedDict()
    for j in rows:
        r = j.record
        shapes.setdefault(r.get("tag") or "%sx%sx%s" % (r["M"], r["N"], r["K"]), []).append(j)
    out = []
    for tag, js in shapes.items():
        meas = [j.measured for j in js]
        pred = [j.predicted for j in js]
        tie = S.top_tie(pred, meas)
        best = max(meas)
        out.append(ShapeRanking(tag, S.spearman(meas, pred),
                                max(collections.Counter(pred).values()), S.best_rank_range(pred, meas),
                                (S.regret(best, min(tie)), S.regret(best, max(tie))), len(tie)))
    return out


@dataclass
class LaunchOrderSummary:
    """Rows of one shape that differ only in groupM, compared in pairs.

    `footprint` of a row is the A rows plus B columns that the tiles resident on
    one XCD touch (reuseTilesM * BM + reuseTilesN * BN, the model's launch-order
    term): the bytes each XCD pulls per K-step are proportional to it."""
    families: int
    violations: int        # pairs whose predictions tie iff their footprints differ
    equal_pairs: int       # pairs with equal footprints (tied by construction)
    equal_spread: list     # their measured difference, % of the faster
    ordered_pairs: int     # pairs with different footprints
    concordant: int        # ... that the model orders as measured
    discordant: list       # (shape, (groupM, footprint, predicted, measured) x 2)


def launch_order_families(rows, hw_path):
    """The reference predicts one number for every swizzle setting (README.md:154);
    here groupM enters through the per-XCD panel count. Checks, over every family
    of rows that differ only in groupM, that two launch orders tie exactly when
    their per-XCD footprints are equal, and how often the model orders the others
    as measured."""
    hw = RM.Hardware(hw_path)
    fams = collections.OrderedDict()
    for j in rows:
        r = j.record
        key = tuple(r[c] for c in ("M", "N", "K", "BM", "BN", "BK", "WM", "WN", "stages")) + (r.get("schedule", "-1"),)
        fams.setdefault(key, []).append(j)
    out = LaunchOrderSummary(0, 0, 0, [], 0, 0, [])
    for key, js in fams.items():
        if len(js) < 2:
            continue
        out.families += 1
        members = []
        for j in js:
            r = j.record
            p = RM.predict(hw, M=int(r["M"]), N=int(r["N"]), K=int(r["K"]), BM=int(r["BM"]), BN=int(r["BN"]),
                           BK=int(r["BK"]), warpM=int(r["WM"]), warpN=int(r["WN"]), stages=int(r["stages"]),
                           regsPerThread=int(r["regsPerThread"]), groupM=int(r["groupM"]),
                           schedule=int(r.get("schedule", "-1") or -1))
            footprint = p["reuseTilesM"] * int(r["BM"]) + p["reuseTilesN"] * int(r["BN"])
            members.append((int(r["groupM"]), footprint, p["predictedTFLOPS"], j.measured))
        for a in range(len(members)):
            for b in range(a + 1, len(members)):
                x, y = members[a], members[b]
                if (x[1] == y[1]) != (x[2] == y[2]):
                    out.violations += 1
                if x[1] == y[1]:
                    out.equal_pairs += 1
                    out.equal_spread.append(abs(x[3] - y[3]) / max(x[3], y[3]) * 100.0)
                    continue
                out.ordered_pairs += 1
                if (x[2] - y[2]) * (x[3] - y[3]) > 0:
                    out.concordant += 1
                else:
                    out.discordant.append((key[:3], x, y))
    hw.close()
    return out


def _mean(xs):
    return sum(xs) / len(xs) if xs else S.NAN


def vendor_ratios(paths):
    """The table's best row against the vendor library on every shape of the
    measured files: [(ratio, (M, N, K), path)], where ratio is the shape's largest
    `tflops` over the median of its rows' `blas_tflops` (ridge-measure times the
    vendor library beside every row, in the same process)."""
    out = []
    for path in paths:
        by = collections.defaultdict(list)
        for r in T.read(path, require=("M", "N", "K", "tflops", "blas_tflops")).records:
            by[(int(r["M"]), int(r["N"]), int(r["K"]))].append(r)
        for shape, rs in sorted(by.items()):
            best = max(float(r["tflops"]) for r in rs)
            out.append((best / S.quantile([float(r["blas_tflops"]) for r in rs], 50), shape, path))
    return out


def print_vendor_ratios(paths):
    ratios = vendor_ratios(paths)
    xs = [x for x, _, _ in ratios]
    lo, hi = min(ratios), max(ratios)
    print("best row against hipBLASLt over %d shapes of %d files" % (len(xs), len(paths)))
    print("  faster on %d; geometric mean %.3fx, median %.3fx" % (
        sum(x > 1 for x in xs), math.exp(_mean([math.log(x) for x in xs])), S.quantile(xs, 50)))
    for name, (x, shape, path) in (("lowest", lo), ("highest", hi)):
        print("  %-8s %.3fx at %dx%dx%d (%s)" % (name, x, *shape, os.path.basename(path)))
    return 0


def report(rows, meta, hw, gate_lines, mape_target, mape_ceiling):
    """Prints the report; returns the list of failed gates."""
    failed = []
    rule = "-" * 74
    print(rule)
    print("ridge cost model against measurement")
    print(rule)
    for k in ("gpu", "cus", "sms", "nominal_clock_mhz", "warmup_seconds", "canary_drift_fraction"):
        if k in meta:
            print("  %-24s %s" % (k, meta[k]))
    print("  %-24s %s\n" % ("hardware model", hw))
    for line in gate_lines:
        print(line)

    errs = [j.abs_pct for j in rows]
    mape = _mean(errs)
    print("absolute error (%d rows)" % len(rows))
    print("  %-22s %8.2f %%   (target <= %.0f%%, ceiling %.0f%%)" % ("MAPE", mape, mape_target, mape_ceiling))
    for name, pct in (("median", 50), ("p90", 90)):
        print("  %-22s %8.2f %%" % (name, S.quantile(errs, pct)))
    print("  %-22s %8.2f %%" % ("max", max(errs)))
    print("  %-22s %+8.2f %%   (negative: the model under-predicts)" % ("mean signed", _mean([j.signed_pct for j in rows])))
    print("\n  largest errors:")
    for j in sorted(rows, key=lambda j: j.abs_pct, reverse=True)[:8]:
        r = j.record
        print("    %5sx%-5sx%-5s %3sx%-3sx%-2s w%sx%s s%s   measured %8.1f  predicted %8.1f  %+7.1f%%" % (
            r["M"], r["N"], r["K"], r["BM"], r["BN"], r["BK"], r["WM"], r["WN"], r["stages"], j.measured,
            j.predicted, j.signed_pct))
    classes = error_by_resident_waves(rows)
    if classes:
        # The wavefront analogue of the reference's 4-active-warp error class
        # (README.md:160).
        print("\n  by resident wavefronts per SIMD and workgroup kind:")
        for (w, kind), (n, a, sg) in sorted(classes.items()):
            print("    %4g waves/SIMD  %-20s %4d rows  MAPE %5.1f%%  signed %+6.1f%%" % (w, kind, n, a, sg))
    print()
    if mape > mape_ceiling:
        failed.append("MAPE %.1f%% is above the %.0f%% ceiling" % (mape, mape_ceiling))

    ranking = rank_shapes(rows)
    print("ranking, per shape (ranges run over predicted ties)")
    print("  %-28s %8s %7s %13s %16s" % ("shape", "rho", "tie", "best at", "regret@1 %"))
    for s in ranking:
        lo, hi = s.best_rank
        rw, rb = s.regret1
        print("  %-28s %8s %7d %13s %16s" % (
            s.tag[:28], "n/a" if s.rho != s.rho else "%.3f" % s.rho, s.largest_tie,
            str(lo) if lo == hi else "%d-%d" % (lo, hi),
            "%.1f" % (rw * 100) if s.top_tie == 1 else "%.1f..%.1f" % (rb * 100, rw * 100)))
    defined = [s.rho for s in ranking if s.rho == s.rho]
    mean_rho = _mean(defined)
    worst = max(s.regret1[0] for s in ranking)
    print("\n  mean rho %.3f over %d shapes (%d without predicted variance)" % (
        mean_rho, len(defined), len(ranking) - len(defined)))
    print("  mean regret@1 %.2f%% (ties broken pessimistically), worst %.2f%%" % (
        _mean([s.regret1[0] for s in ranking]) * 100, worst * 100))
    print("  largest group of equal predictions: %d configs\n" % max(s.largest_tie for s in ranking))
    if rows and "schedule" in rows[0].record:
        lo = launch_order_families(rows, hw)
        print("launch order (rows that differ only in groupM): %d families" % lo.families)
        print("  %d pairs with equal per-XCD footprints, all tied; measured difference median %.2f%%, max %.2f%%" % (
            lo.equal_pairs, S.quantile(lo.equal_spread, 50) if lo.equal_spread else S.NAN,
            max(lo.equal_spread) if lo.equal_spread else S.NAN))
        print("  %d pairs with different footprints, ordered as measured: %d (%.0f%%)" % (
            lo.ordered_pairs, lo.concordant, 100.0 * lo.concordant / lo.ordered_pairs if lo.ordered_pairs else 0))
        print("  ties that do not follow the footprint: %d\n" % lo.violations)
        if lo.violations:
            failed.append("%d groupM pairs tie without equal footprints, or differ with them" % lo.violations)
    labels = collections.Counter(j.record["pred_bottleneck"] for j in rows)
    print("predicted bottleneck labels: %s" % ", ".join("%s %d" % kv for kv in labels.most_common()))
    print("counter cross-check: python -m ridge_amd.labelcheck\n")
    print(rule)
    print("MAPE %.2f%%, mean Spearman %.3f, worst regret@1 %.2f%%" % (mape, mean_rho, worst * 100))
    return failed


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--measured", default=os.path.join(ROOT, "data", "measured", "mi355x.csv"))
    ap.add_argument("--registered", default=os.path.join(ROOT, "data", "sweep", "mi355x-registered.csv"))
    ap.add_argument("--hw", default=os.path.join(ROOT, "data", "hardware", "mi355x.json"))
    ap.add_argument("--predict-bin", default=RM.PREDICT_BIN, help="the ridge-predict executable")
    ap.add_argument("--max-mape", type=float, default=10.0)
    ap.add_argument("--fail-mape", type=float, default=15.0)
    ap.add_argument("--no-table-gate", action="store_true",
                    help="skip the registered cross-product gate (e.g. for another GPU's sweep)")
    ap.add_argument("--vendor", nargs="+", metavar="MEASURED_CSV",
                    help="only compare the best row with hipBLASLt over the shapes of these files")
    args = ap.parse_args(argv)
    if args.vendor:
        return print_vendor_ratios(args.vendor)
    try:
        meta = T.read(args.measured).meta
        rows = join(args.measured, args.hw, args.predict_bin)
        if not rows:
            raise T.TableError(args.measured, 0, "no measured rows")
        gate_lines, failed = [], []
        if not args.no_table_gate:
            shapes = T.read_shapes(args.registered)
            keys = kernel_table_keys()
            absent, unexpected = registered_gate([j.record for j in rows], shapes, keys)
            gate_lines.append("registered: %d shapes x %d kernels = %d rows; measured %d rows" % (
                len(shapes), len(keys), len(shapes) * len(keys), len(rows)))
            if absent or unexpected:
                gate_lines.append("  %d registered rows were not measured, %d measured rows were not registered"
                                  % (len(absent), len(unexpected)))
                gate_lines += ["    absent: %s" % (a,) for a in sorted(absent)[:5]]
                failed.append("the measured rows are not the registered cross product")
            else:
                gate_lines.append("  the measured rows are exactly the registered cross product")
            gate_lines.append("")
    except (T.TableError, RuntimeError) as e:
        sys.exit(str(e))
    failed += report(rows, meta, args.hw, gate_lines, args.max_mape, args.fail_mape)
    for f in failed:
        print("  FAILED: %s" % f)
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
