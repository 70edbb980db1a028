"""The calibration driver (no GPU): the committed hardware JSON is what the
committed benchmark log derives, and the driver refuses a log whose constants are
out of band or missing."""
import os

import pytest

from ridge_amd import calibrate

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LOG = os.path.join(ROOT, "data", "hardware", "mi355x-calibration.txt")
JSON = os.path.join(ROOT, "data", "hardware", "mi355x.json")


def test_committed_json_rederives_from_the_committed_log(tmp_path):
    out = tmp_path / "hw.json"
    assert calibrate.main(["--from-log", LOG, "--out", str(out)]) == 0
    assert out.read_text() == open(JSON).read()


def _log_with(tmp_path, old, new):
    text = open(LOG).read()
    assert old in text
    p = tmp_path / "log.txt"
    p.write_text(text.replace(old, new))
    return str(p)


def test_a_clock_ratio_below_the_full_chip_clock_is_refused(tmp_path):
    """A partly busy chip clocking slower than the full chip means the sweep
    measured something else: the driver refuses and writes nothing."""
    line = [l for l in open(LOG) if l.startswith("CAL_RESULT clockRatioHalfCus")][0]
    log = _log_with(tmp_path, line, "CAL_RESULT clockRatioHalfCus 0.5\n")
    out = tmp_path / "hw.json"
    assert calibrate.main(["--from-log", log, "--out", str(out)]) == 1
    assert not out.exists()


def test_a_log_without_the_per_operand_lds_rates_is_refused(tmp_path):
    line = [l for l in open(LOG) if l.startswith("CAL_RESULT ldsBTrReadBytesPerCycle")][0]
    log = _log_with(tmp_path, line, "")
    with pytest.raises(SystemExit, match="ldsBTrReadBytesPerCycle"):
        calibrate.main(["--from-log", log, "--out", str(tmp_path / "hw.json")])
