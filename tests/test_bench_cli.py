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
