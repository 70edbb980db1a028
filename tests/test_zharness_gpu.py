"""The two native harnesses on the GPU: ridge-check (the checker's self-test,
every variant on the reference's six correctness shapes, throughput at 4096^3
against hipBLASLt with the 0.80 floor) and ridge-measure on a two-shape sweep
(the measured-CSV contract: one row per dividing variant, the registered
columns, the row's schedule). Collected after the GEMM parity tests."""
import csv
import os
import subprocess

import pytest

from ridge_amd import gemm as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "ridge_amd", "bin")


@pytest.mark.gpu
def test_ridge_check_passes():
    print("step: ridge-check", flush=True)
    proc = subprocess.run([os.path.join(BIN, "ridge-check")], cwd=ROOT, capture_output=True, text=True,
                          timeout=300)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert "FAIL" not in proc.stdout.replace("must FAIL", "")


@pytest.mark.gpu
def test_ridge_measure_writes_the_registered_columns(tmp_path):
    sweep = tmp_path / "sweep.csv"
    sweep.write_text("# two shapes for the harness test\n# M,N,K,tag,rationale\n"
                     "1024,1024,1024,t-1024cube,every variant divides it\n"
                     "2048,512,256,t-2048x512x256,the 256-wide tiles do not divide N\n")
    out = tmp_path / "measured.csv"
    print("step: ridge-measure", flush=True)
    proc = subprocess.run([os.path.join(BIN, "ridge-measure"), str(sweep), str(out), "--allow-skip",
                           "--warmup-seconds", "1", "--settle-seconds", "0.05"],
                          cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    lines = [l for l in out.read_text().splitlines() if not l.startswith("#")]
    rows = list(csv.DictReader(lines))
    cols = ["M", "N", "K", "tag", "BM", "BN", "BK", "WM", "WN", "stages", "groupM", "regsPerThread", "smemBytes",
            "threads", "tflops", "blas_tflops", "fraction_of_blas", "canary_tflops", "ms", "iters", "schedule"]
    assert list(rows[0].keys()) == cols
    table = {(v.BM, v.BN, v.BK, v.WM, v.WN, v.stages, v.groupM): v for v in G.variants()}
    for (M, N, K) in ((1024, 1024, 1024), (2048, 512, 256)):
        got = [r for r in rows if (int(r["M"]), int(r["N"]), int(r["K"])) == (M, N, K)]
        want = [v for v in G.variants() if v.divides(M, N, K)]
        assert len(got) == len(want) and want
        for r in got:
            v = table[tuple(int(r[c]) for c in ("BM", "BN", "BK", "WM", "WN", "stages", "groupM"))]
            assert int(r["schedule"]) == v.schedule
            assert float(r["tflops"]) > 0 and float(r["blas_tflops"]) > 0 and float(r["canary_tflops"]) > 0
            assert float(r["ms"]) > 0 and int(r["iters"]) > 0


@pytest.mark.gpu
def test_ridge_measure_times_registered_launch_plans(tmp_path):
    """--plans: one single-row plan and one row split of 1536 x 1536 x 512 (the
    64x64 row on 1024 rows, the 128x128 persistent row on the other 512; any
    split the two rows divide is timed, whether or not the planner would choose
    it): both timed, hipBLASLt read once for the shape, and the plan's columns
    repeated with both rows' schedules."""
    plans = tmp_path / "plans.csv"
    plans.write_text("# two plans for the harness test\n"
                     "M,N,K,tag,BM,BN,BK,WM,WN,stages,groupM,body_rows,"
                     "tail_BM,tail_BN,tail_BK,tail_WM,tail_WN,tail_stages,tail_groupM,role\n"
                     "1536,1536,512,t,256,256,32,128,64,3,4,1536,0,0,0,0,0,0,0,anchor\n"
                     "1536,1536,512,t,64,64,64,32,32,4,8,1024,128,128,64,64,64,4,8,split\n")
    out = tmp_path / "measured.csv"
    print("step: ridge-measure --plans", flush=True)
    proc = subprocess.run([os.path.join(BIN, "ridge-measure"), "--plans", str(plans), str(out),
                           "--warmup-seconds", "1", "--settle-seconds", "0.05"],
                          cwd=ROOT, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-2000:]
    assert proc.stdout.count("1536x1536x512  hipBLASLt") == 1
    rows = list(csv.DictReader(l for l in out.read_text().splitlines() if not l.startswith("#")))
    assert [int(r["body_rows"]) for r in rows] == [1536, 1024]
    assert [int(r["schedule"]) for r in rows] == [1, 0] and [int(r["tail_schedule"]) for r in rows] == [-1, 2]
    assert rows[0]["blas_tflops"] == rows[1]["blas_tflops"]
    for r in rows:
        assert float(r["tflops"]) > 0 and float(r["ms"]) > 0 and int(r["iters"]) > 0
