"""Regret and ranking statistics (no GPU): closed forms and hand-made cases,
including the stable tie order the pruner depends on
(tools/ridge-autotune.py:93-104, bench/validate.py:36-184)."""
import csv
import os

import pytest

from ridge_amd import autotune as AT
from ridge_amd import validate as V

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")


def test_regret_at_k_hand_case():
    # shape a: best measured 100 is predicted 3rd; shape b: predicted top is best.
    shapes = {
        "a": [(50.0, 80.0), (40.0, 90.0), (30.0, 100.0)],
        "b": [(10.0, 70.0), (9.0, 60.0), (8.0, 50.0)],
    }
    mean1, max1, hits1, per1 = AT.regret_at_k(shapes, 1)
    assert per1 == [pytest.approx(20.0), 0.0] and hits1 == 1
    assert mean1 == pytest.approx(10.0) and max1 == pytest.approx(20.0)
    mean2, _, hits2, per2 = AT.regret_at_k(shapes, 2)
    assert per2 == [pytest.approx(10.0), 0.0] and hits2 == 1
    mean3, _, hits3, _ = AT.regret_at_k(shapes, 3)
    assert mean3 == 0.0 and hits3 == 2


def test_ties_break_by_table_order():
    # Three configs tie on prediction; a stable sort keeps input order, so k=1
    # picks the first row (measured 60), not the best of the tie (90).
    shapes = {"s": [(100.0, 60.0), (100.0, 90.0), (100.0, 75.0), (50.0, 95.0)]}
    _, _, _, per = AT.regret_at_k(shapes, 1)
    assert per == [pytest.approx((95 - 60) / 95 * 100)]
    _, _, _, per = AT.regret_at_k(shapes, 2)
    assert per == [pytest.approx((95 - 90) / 95 * 100)]
    _, _, _, per = AT.regret_at_k(shapes, 4)
    assert per == [0.0]


def test_average_ranks_and_spearman_textbook():
    assert V.average_ranks([10, 20, 20, 30]) == [1.0, 2.5, 2.5, 4.0]
    assert V.spearman([1, 2, 3, 4], [10, 20, 30, 40]) == pytest.approx(1.0)
    assert V.spearman([1, 2, 3, 4], [4, 3, 2, 1]) == pytest.approx(-1.0)
    # Constant prediction has no variance: reported as nan, not 0.
    r = V.spearman([1, 2, 3], [5, 5, 5])
    assert r != r
    # Classic example with ties: x=[1,2,3,4,5], y=[2,1,4,3,5]: d^2 sum = 4 -> 1 - 6*4/(5*24) = 0.8
    assert V.spearman([1, 2, 3, 4, 5], [2, 1, 4, 3, 5]) == pytest.approx(0.8)


def test_rank_and_regret_bounds_over_ties():
    rows = [{"pred_tflops": p, "tflops": m} for p, m in [(9, 50), (9, 100), (8, 70), (7, 60)]]
    assert V.rank_bounds(rows) == (1, 2)            # best (100) sits in a 2-way top tie
    worst, best, n = V.regret_bounds(rows)
    assert n == 2 and worst == pytest.approx(0.5) and best == 0.0


def test_cross_product_gate_detects_missing_and_extra():
    reg = [(256, 256, 64)]
    variants = [(128, 128, 32, 64, 64, 2, 8), (64, 64, 32, 32, 32, 4, 8)]
    def row(v):
        return dict(zip(("M", "N", "K", "BM", "BN", "BK", "WM", "WN", "stages", "groupM"), map(str, (256, 256, 64) + v)))
    missing, extra = V.cross_product_gate([row(variants[0])], reg, variants)
    assert missing == {(256, 256, 64) + variants[1]} and not extra
    missing, extra = V.cross_product_gate([row(variants[0]), row(variants[1]), row((256, 256, 64, 128, 128, 2, 8))],
                                          reg, variants)
    assert not missing and extra == {(256, 256, 64, 256, 256, 64, 128, 128, 2, 8)}


def test_autotune_end_to_end_on_reference_a100_sweep():
    """The reference's own sweep and calibrated constants, through the model CLI:
    the pruner finds the exhaustive best on every shape by k = 10."""
    table, total, nshapes, per_shape = AT.evaluate(os.path.join(GOLD, "a100_measured.csv"),
                                                   os.path.join(GOLD, "a100-sxm4-40gb.json"))
    assert (total, nshapes, per_shape) == (336, 14, 24)
    k10 = [r for r in table if r["k"] == 10][0]
    assert k10["mean_regret"] == 0.0 and k10["hits"] == 14
    k1 = [r for r in table if r["k"] == 1][0]
    assert 0.0 < k1["mean_regret"] < 15.0


def test_measured_mi355x_sweep_is_the_registered_cross_product():
    """The committed MI355X sweep covers exactly shapes x table (the measurement
    integrity gate of bench/validate.py:136-156)."""
    path = os.path.join(ROOT, "data", "measured", "mi355x.csv")
    rows = list(csv.DictReader(l for l in open(path) if not l.startswith("#")))
    missing, extra = V.cross_product_gate(rows, V.load_registered(os.path.join(ROOT, "data", "sweep",
                                                                              "mi355x-registered.csv")),
                                          V.load_variant_table())
    assert not missing and not extra


@pytest.mark.parametrize("name", ["mi355x.csv", "mi355x-replicate.csv"])
def test_mi355x_pruner_meets_the_target_on_each_measurement(name):
    """The calibrated model prunes the MI355X sweep to within the BASELINE target
    (mean regret <= 2% at k = 10) on the committed measurement and on an
    independent re-measurement taken on another box; both cover the registered
    cross product."""
    path = os.path.join(ROOT, "data", "measured", name)
    rows = list(csv.DictReader(l for l in open(path) if not l.startswith("#")))
    missing, extra = V.cross_product_gate(rows, V.load_registered(os.path.join(ROOT, "data", "sweep",
                                                                              "mi355x-registered.csv")),
                                          V.load_variant_table())
    assert not missing and not extra
    table, total, nshapes, per_shape = AT.evaluate(path, os.path.join(ROOT, "data", "hardware", "mi355x.json"))
    assert (total, nshapes) == (336, 14)
    k10 = [r for r in table if r["k"] == 10][0]
    assert k10["mean_regret"] <= 2.0


def test_error_classes_by_resident_waves_hand_case():
    """Two 4-wave rows with two resident workgroups (2 waves per SIMD) and one
    8-wave ping-pong row with one (2 per SIMD, its own class): per-class mean of
    |err| and of signed err."""
    rows = [
        dict(BM="128", BN="128", WM="64", WN="64", pred_ctas_per_sm="2", schedule="0", _abs=10.0, _signed=10.0),
        dict(BM="128", BN="128", WM="64", WN="64", pred_ctas_per_sm="2", schedule="0", _abs=20.0, _signed=-20.0),
        dict(BM="256", BN="256", WM="128", WN="64", pred_ctas_per_sm="1", schedule="1", _abs=5.0, _signed=5.0),
    ]
    got = V.error_by_resident_waves(rows)
    assert got == {(2.0, "4-wave uniform"): (2, 15.0, -5.0), (2.0, "8-wave ping-pong"): (1, 5.0, 5.0)}
    assert V.error_by_resident_waves([dict(BM="1")]) == {}
