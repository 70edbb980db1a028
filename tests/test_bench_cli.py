"""bench.py's contract on a machine without a GPU: a request for more than one GPU
exits with a message (the build measures one device) and no GPU call."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = subprocess.run([sys.executable, "bench.py", "--gpus", "2", "--steps", "1", "--warmup", "0"], cwd=ROOT,
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in (proc.stdout + proc.stderr)


def test_window_statistics():
    """bench.py reports the middle of its timed windows, with the fastest and
    slowest, as TFLOP/s from per-launch milliseconds."""
    sys.path.insert(0, ROOT)
    import bench
    assert bench.middle([3.0, 1.0, 2.0]) == 2.0 and bench.middle([4.0, 1.0, 2.0, 3.0]) == 2.5
    flops = 2.0e12  # 2 TFLOP per launch: 1 ms per launch is 2000 TFLOP/s
    s = bench.window_summary(flops, [1.0, 2.0, 1.25, 1.0, 4.0])
    assert s["tflops"] == 1600.0 and s["max"] == 2000.0 and s["min"] == 500.0 and s["windows"] == 5
    assert s["range_pct"] == 93.75
