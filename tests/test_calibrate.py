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


# Constants every calibration here measured the same way, and those only the
# current benches measure (the ping-pong skeleton's refill carries random
# halves; the kernel-boundary section of cal-latency).
SAME_METHOD_KEYS = ["clockHz", "hbmBytesPerSec", "hbmWriteBytesPerSec", "mallRefillBytesPerSec",
                    "l2HitBytesPerCycle", "smemBytesPerCycle", "mmaCyclesPerInst"]
CURRENT_METHOD_KEYS = ["loadedClockRatio", "launchSeconds"]


@pytest.mark.parametrize("box,keys", [("box2", SAME_METHOD_KEYS),
                                      ("box3", SAME_METHOD_KEYS + CURRENT_METHOD_KEYS)])
def test_other_box_calibrations_leave_the_rankings_unchanged(tmp_path, box, keys):
    """Whole calibration runs on other boxes: mi355x-box2 with the benches as they
    were before the random-data refill and the launch constants, mi355x-box3 with
    the current benches but for the kernel-boundary section. Each JSON re-derives
    from its log, holds no key the committed one lacks, its constants measured the
    same way sit within 6% of the committed ones, and the pruner's regret at
    k = 1 and k = 10 on the in-sample sweep, its replicate and the fourth
    held-out sweep is the same to the hundredth. Those runs predate the MALL
    write measurement, so the committed constant and its term are added to each
    for the comparison."""
    import json
    from ridge_amd import autotune as AT
    hw = os.path.join(ROOT, "data", "hardware")
    log2, json2 = os.path.join(hw, "mi355x-calibration-%s.txt" % box), os.path.join(hw, "mi355x-%s.json" % box)
    out = tmp_path / "hw2.json"
    assert calibrate.main(["--from-log", log2, "--out", str(out)]) == 0
    assert out.read_text() == open(json2).read()
    a, b = json.load(open(JSON)), json.load(open(json2))
    assert set(b) <= set(a)
    for key in keys:
        assert abs(b[key] / a[key] - 1.0) < 0.06, key
    later = {k: a[k] for k in ("mallWriteModel", "mallWriteBytesPerSec")}
    assert not set(later) & set(b)
    b.update(later)
    with_later = tmp_path / "hw2-mall-write.json"
    with_later.write_text(json.dumps(b))
    measured = os.path.join(ROOT, "data", "measured")
    for name in ("mi355x.csv", "mi355x-replicate.csv", "mi355x-heldout4.csv"):
        sweep = os.path.join(measured, name)
        ref = {r["k"]: (round(r["mean_regret"], 2), round(r["max_regret"], 2))
               for r in AT.evaluate(sweep, JSON, ks=(1, 10))[0]}
        new = {r["k"]: (round(r["mean_regret"], 2), round(r["max_regret"], 2))
               for r in AT.evaluate(sweep, str(with_later), ks=(1, 10))[0]}
        assert ref == new, name
