"""Launch plans ranked by the cost model (ridge_amd/rowsplit.py) and the plan list
ridge-measure times (--plans): CPU only. The model's figures come from the
committed calibration; the ranking, registration and scoring arithmetic are
checked against hand-built inputs."""
import os
import subprocess

import pytest

from ridge_amd import gemm as G
from ridge_amd import model as RM
from ridge_amd import rowsplit as R
from ridge_amd import tables as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HW = os.path.join(ROOT, "data", "hardware", "mi355x.json")
MEASURE = os.path.join(ROOT, "ridge_amd", "bin", "ridge-measure")
S3 = (256, 256, 32, 128, 64, 3, 4)
P128 = (128, 128, 64, 64, 64, 4, 8)


@pytest.fixture(scope="module")
def ranker():
    return R.Ranker(HW)


def _model_seconds(key, M, N, K):
    v = G.variant(G.find_variant(*key))
    p = RM.predict(RM.Hardware(HW), M=M, N=N, K=K, BM=v.BM, BN=v.BN, BK=v.BK, warpM=v.WM, warpN=v.WN,
                   stages=v.stages, regsPerThread=v.regsPerThread, groupM=v.groupM, schedule=v.schedule)
    return 2.0 * M * N * K / (p["predictedTFLOPS"] * 1e12)


def test_a_split_is_priced_as_its_two_launches(ranker):
    """6144 x 3072 x 6144: the model's first plan is the 256x256 s3 row on the 5376
    rows of one round plus the 128x128 persistent row on the last 768, and its
    time is the two launches' predicted times added, each a prediction of its own
    sub-shape."""
    plans = ranker.rank(6144, 3072, 6144)
    first = plans[0]
    assert first.split and first.rows == 5376
    assert G.variant(first.body).key() == S3 and G.variant(first.tail).key() == P128
    want = _model_seconds(S3, 5376, 3072, 6144) + _model_seconds(P128, 768, 3072, 6144)
    assert first.seconds == pytest.approx(want, rel=1e-12)
    assert sum(not p.split for p in plans) == 24
    assert all(a.seconds <= b.seconds for a, b in zip(plans, plans[1:]))
    # 4096^3 is one whole round of 256x256 tiles: the 256x256 rows offer no split.
    assert not any(p.split and G.variant(p.body).BM == 256 and G.variant(p.body).BN == 256
                   for p in ranker.rank(4096, 4096, 4096))


def test_distinct_splits_keep_one_body_per_split_point_and_tail(ranker):
    got = R.distinct_splits(ranker, 6144, 3072, 6144, 5)
    assert len(got) == 5
    assert len({(p.rows, p.tail) for p in got}) == 5
    every = ranker.splits(6144, 3072, 6144)
    for p in got:
        same = [q for q in every if (q.rows, q.tail) == (p.rows, p.tail)]
        assert p.seconds == min(q.seconds for q in same)
    # Under one round for every row: no split, so the shape is not registered.
    assert R.distinct_splits(ranker, 256, 256, 64, 5) == []


def _sweep_csv(path, rows):
    cols = ["M", "N", "K", "tag"] + list(R.KEY) + ["tflops"]
    recs = [dict(zip(["M", "N", "K", "tag"], s[:3] + ("t",)), **dict(zip(R.KEY, key)), tflops=tf)
            for s, key, tf in rows]
    T.write(str(path), cols, recs)


def test_register_anchor_model_single_and_splits(tmp_path, ranker):
    """The anchor is the row measured fastest in the sweep CSVs (over two files),
    the model's best single row follows when it is another row, then the distinct
    splits; a shape with no split is left out."""
    a, b = tmp_path / "a.csv", tmp_path / "b.csv"
    _sweep_csv(a, [((6144, 3072, 6144), P128, 1000.0), ((6144, 3072, 6144), S3, 900.0),
                   ((256, 256, 64), (64, 64, 64, 32, 32, 4, 8), 50.0)])
    _sweep_csv(b, [((6144, 3072, 6144), S3, 1001.0)])
    recs = R.register([(6144, 3072, 6144, "x"), (256, 256, 64, "small")], [str(a), str(b)], ranker, 3)
    assert {r["tag"] for r in recs} == {"x"}
    roles = [r["role"] for r in recs]
    top_single = min(ranker.singles(6144, 3072, 6144), key=lambda p: p.seconds)
    assert roles[0] == "anchor" and tuple(recs[0][c] for c in R.KEY) == S3 and recs[0]["body_rows"] == 6144
    assert all(recs[0]["tail_" + c] == 0 for c in R.KEY)
    if G.variant(top_single.body).key() != S3:
        assert roles[1] == "model_single"
    assert roles[-3:] == ["model_split_1", "model_split_2", "model_split_3"]


def test_score_gain_and_regrets_by_hand(tmp_path, ranker):
    """Hand-set measured rates for a registered shape: the best single row 1000,
    the model's first split 1200 and the other splits 1100, so the gain is 1.2,
    a model that picks the split has regret 0, one limited to single rows has
    (1200 - its row's rate) / 1200, and the hipBLASLt ratio is over the median
    comparator reading."""
    M, N, K = 6144, 3072, 6144
    a = tmp_path / "a.csv"
    _sweep_csv(a, [((M, N, K), P128, 1000.0)])
    recs = R.register([(M, N, K, "x")], [str(a)], ranker, 3)
    plans = tmp_path / "plans.csv"
    T.write(str(plans), R.PLAN_COLUMNS, recs)
    rate = {"anchor": 1000.0, "model_single": 950.0, "model_split_1": 1200.0}
    meas = []
    for r in recs:
        m = dict(r)
        m["tflops"] = rate.get(r["role"], 1100.0)
        m["blas_tflops"] = 1050.0
        meas.append(m)
    out = tmp_path / "measured.csv"
    T.write(str(out), R.PLAN_COLUMNS + ["tflops", "blas_tflops"], meas)
    (row,) = R.score(str(plans), str(out), ranker)
    assert row["best_single"] == 1000.0 and row["best_split"] == 1200.0
    assert row["gain"] == pytest.approx(1.2)
    assert row["model_picks_split"] and row["regret_with_splits"] == 0.0
    first_single = next(p for p in ranker.rank(M, N, K) if not p.split)
    single_rate = 1000.0 if G.variant(first_single.body).key() == P128 else 950.0
    assert row["regret_singles"] == pytest.approx((1200.0 - single_rate) / 1200.0 * 100)
    assert row["best_vs_blas"] == pytest.approx(1200.0 / 1050.0)
    # A registered plan without a measurement is refused.
    T.write(str(out), R.PLAN_COLUMNS + ["tflops", "blas_tflops"], meas[:-1])
    with pytest.raises(ValueError, match="not measured"):
        R.score(str(plans), str(out), ranker)


PLAN_HEADER = ("M,N,K,tag,BM,BN,BK,WM,WN,stages,groupM,body_rows,"
               "tail_BM,tail_BN,tail_BK,tail_WM,tail_WN,tail_stages,tail_groupM\n")


@pytest.mark.parametrize("record,message", [
    ("6144,3072,6144,x,256,256,32,128,64,3,4,5300,128,128,64,64,64,4,8", "a split needs"),
    ("6144,3072,6144,x,256,256,32,128,64,3,4,6144,128,128,64,64,64,4,8", "zero tail key"),
    ("6144,3072,6144,x,256,256,32,128,64,9,4,5376,128,128,64,64,64,4,8", "body key is not a row"),
    ("6144,3072,6144,x,256,256,32,128,64,3,4,5376,128,128,64,64,64,9,8", "tail key is not a row"),
    ("6000,3072,6144,x,256,256,32,128,64,3,4,6000,0,0,0,0,0,0,0", "does not divide"),
    ("6144,3072,6144,x,256,256,32,128,64,3,4,abc,0,0,0,0,0,0,0", "must be integers"),
])
def test_ridge_measure_refuses_a_bad_plan_before_touching_the_device(tmp_path, record, message):
    plans = tmp_path / "plans.csv"
    plans.write_text("# one plan\n" + PLAN_HEADER + record + "\n")
    proc = subprocess.run([MEASURE, "--plans", str(plans), str(tmp_path / "out.csv")], capture_output=True,
                          text=True, timeout=60)
    assert proc.returncode == 2, proc.stdout + proc.stderr
    assert message in proc.stderr and "plans.csv:3" in proc.stderr
    assert not (tmp_path / "out.csv").exists()


def test_ridge_measure_refuses_a_plan_list_without_a_column(tmp_path):
    plans = tmp_path / "plans.csv"
    plans.write_text(PLAN_HEADER.replace(",body_rows", "") + "1,1,1,x,1,1,1,1,1,1,1,0,0,0,0,0,0,0\n")
    proc = subprocess.run([MEASURE, "--plans", str(plans), str(tmp_path / "out.csv")], capture_output=True,
                          text=True, timeout=60)
    assert proc.returncode == 2 and "no column body_rows" in proc.stderr


SWEEPS = ["data/sweep/mi355x-heldout-registered.csv"] + [
    "data/sweep/mi355x-heldout%d-registered.csv" % i for i in range(2, 8)] + ["data/sweep/mi355x-registered.csv"]
MEASURED = ["data/measured/mi355x.csv", "data/measured/mi355x-heldout.csv"] + [
    "data/measured/mi355x-heldout%d.csv" % i for i in range(2, 8)]


def test_registered_plan_list_regenerates_from_the_committed_inputs(tmp_path):
    """data/sweep/mi355x-rowsplit-plans.csv is what `register` writes from the
    committed sweeps, measured CSVs and frozen constants: 543 plans on 89 shapes,
    5 distinct splits on 77 of them and 3 on 12, the model's best single row
    beside the anchor on 33."""
    out = tmp_path / "plans.csv"
    argv = ["register", "--hw", "data/sweep/mi355x-rowsplit-hw.json", "--sweeps",
            ",".join(os.path.join(ROOT, p) for p in SWEEPS), "--measured",
            ",".join(os.path.join(ROOT, p) for p in MEASURED), "--out", str(out)]
    cwd = os.getcwd()
    os.chdir(ROOT)
    try:
        assert R.main(argv) == 0
    finally:
        os.chdir(cwd)
    committed = T.read(os.path.join(ROOT, "data", "sweep", "mi355x-rowsplit-plans.csv")).records
    assert T.read(str(out)).records == committed
    assert len(committed) == 543
    shapes = {(r["M"], r["N"], r["K"]) for r in committed}
    assert len(shapes) == 89
    per = [sum(r["role"].startswith("model_split") for r in committed if (r["M"], r["N"], r["K"]) == s)
           for s in shapes]
    assert sorted(per).count(5) == 77 and sorted(per).count(3) == 12
    assert sum(r["role"] == "model_single" for r in committed) == 33


def test_registered_row_split_measurement_figures():
    """The registered measurement (data/sweep/mi355x-rowsplit.md) scored with its
    frozen constants: a split pays on three shapes; C1 (every split the model picks
    beats the single row) fails, 3 of 5; C2 (splits among the candidates lower the
    model's mean regret) passes, 1.40% against 1.73%."""
    ranker = R.Ranker(os.path.join(ROOT, "data", "sweep", "mi355x-rowsplit-hw.json"))
    rows = R.score(os.path.join(ROOT, "data", "sweep", "mi355x-rowsplit-plans.csv"),
                   os.path.join(ROOT, "data", "measured", "mi355x-rowsplit.csv"), ranker)
    assert len(rows) == 89
    wins = sorted(((r["M"], r["N"], r["K"]), round(r["gain"], 3)) for r in rows if r["gain"] > 1.05)
    assert wins == [((6144, 3072, 6144), 1.164), ((12288, 1536, 6144), 1.171), ((12288, 3072, 3072), 1.055)]
    assert sum(r["gain"] > 1.01 for r in rows) == 3
    picks = {(r["M"], r["N"], r["K"]): r for r in rows if r["model_picks_split"]}
    assert sorted(picks) == [(1536, 6144, 2048), (5120, 5120, 3072), (6144, 3072, 6144), (12288, 1536, 6144),
                             (12288, 3072, 3072)]
    assert sum(r["regret_with_splits"] == 0.0 for r in picks.values()) == 3
    assert picks[(5120, 5120, 3072)]["regret_with_splits"] == pytest.approx(13.258, abs=1e-3)
    assert picks[(1536, 6144, 2048)]["regret_with_splits"] == pytest.approx(8.16, abs=1e-2)
    mean = lambda xs: sum(xs) / len(xs)
    assert mean([r["regret_with_splits"] for r in rows]) == pytest.approx(1.398, abs=1e-3)
    assert mean([r["regret_singles"] for r in rows]) == pytest.approx(1.729, abs=1e-3)
    assert max(r["regret_singles"] for r in rows) == pytest.approx(20.037, abs=1e-3)
    assert sum(r["best_vs_blas"] > 1 for r in rows) == 89 and sum(r["best_single_vs_blas"] > 1 for r in rows) == 86
