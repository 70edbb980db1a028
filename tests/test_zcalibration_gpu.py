"""The four calibration microbenchmarks on the GPU, through the driver in --check
mode (band checks and repeat stability; nothing is written), plus the invariants
of the figures that are counted in shader cycles and so do not move with the
box's loaded clock:

  * eight waves reading the headline tile's fragments take A bytes / the A rate +
    B bytes / the transposing-read rate, from the rates measured in the same run;
  * the ping-pong skeleton runs at its MFMA time (the schedule hides the reads);
  * reads served by the XCDs' L2s arrive at 64 B per cycle per CU."""
import os
import subprocess
import sys

import pytest

from ridge_amd import calibrate

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_calibration_benchmarks_are_in_band_and_consistent(tmp_path):
    """Every benchmark runs and reports its constants, every constant is inside the
    driver's sanity band, and the cycle-counted figures agree with each other.
    The driver's repeat-stability gate decides whether a run may be written into
    the hardware JSON; it is not applied here, because the wall-clock figures
    (HBM bytes per second) follow the box's power state from repeat to repeat."""
    log = tmp_path / "cal.txt"
    print("step: python -m ridge_amd.calibrate --check", flush=True)
    proc = subprocess.run([sys.executable, "-u", "-m", "ridge_amd.calibrate", "--check", "--log", str(log)],
                          cwd=ROOT, capture_output=True, text=True, timeout=300)
    text = log.read_text()
    res = calibrate.parse_results(text)
    missing = [k for k in calibrate.REQUIRED_KEYS if k not in res]
    assert not missing, (missing, proc.stdout[-3000:], proc.stderr[-2000:])
    assert calibrate.band_check(res, calibrate.SPECS["gfx950"]), proc.stdout[-3000:]
    tS = 8 * (8 * 1024.0 / res["ldsAReadBytesPerCycle"] + 8 * 512.0 / res["ldsBTrReadBytesPerCycle"])
    assert res["pingPongReadCycles"] == pytest.approx(tS, rel=0.03)
    tC = 8 * 32 * res["mmaCyclesPerInst"]
    assert res["pingPongMfmaCycles"] == pytest.approx(tC, rel=0.03)
    assert res["pingPongStepCycles"] <= 1.03 * max(res["pingPongMfmaCycles"], res["pingPongReadCycles"])
    assert res["pingPongRefillStepCycles"] <= 1.03 * res["pingPongMfmaCycles"]
    assert res["l2HitBytesPerCycle"] == pytest.approx(64.0 * 256, rel=0.05)
