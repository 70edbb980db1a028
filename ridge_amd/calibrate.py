"""Runs the four calibration microbenchmarks and writes the hardware JSON.

    python -m ridge_amd.calibrate [--binary-dir ridge_amd/bin] [--out data/hardware/mi355x.json] [--check]
    python -m ridge_amd.calibrate --from-log data/hardware/mi355x-calibration.txt   # re-derive, no GPU

Counterpart of the reference's bench/calibrate/run-calibration.py:29-159. The
constants come from the benchmarks; the datasheet figures below are independent
cross-checks that catch a broken benchmark, never sources of a value. With
--check nothing is written and the exit code says whether every constant is in
band. A constant out of band, or a benchmark reporting unstable repeats, refuses
the write.

MI355X differences from the reference driver:
  * clockHz is the loaded engine clock MEASURED by cal-mma (shader-clock cycles
    against the constant 100 MHz counter), not a pinned constant, because this
    machine's clocks cannot be locked;
  * the compute band is checked on the peak implied at the nominal clock (what
    the cycle count alone says), the loaded-clock figure is reported beside it;
  * the JSON carries the CDNA4 target description ("arch": "gfx950") and the
    extra measured keys (MALL bandwidth, LDS control and per-pattern rates);
  * the chip is power-limited, so cal-mma also measures the loaded clock with
    1/2 .. 1/16 of the CUs busy (clockRatio*: the model's clockModel 1), the
    per-operand LDS rates feed ldsReadModel 1, and cal-hbm-bw's L2-resident read
    (l2HitBytesPerCycle) feeds l2StreamModel 1;
  * the MALL's capacity (datasheet) with the calibrated refill rate feeds
    mallReuseModel 1: when A and B fit, re-fetches of their panels are MALL hits;
  * cal-smem-bw's ping-pong skeleton figures (reads under MFMAs, with and without
    the GEMM's direct-to-LDS refill) are kept in the JSON as a record, and the ratio
    of its clock with the refill to its clock with MFMAs alone is loadedClockRatio
    (powerModel 1); its free-running mode gives freeRunningOverlap
    (uniformOverlapModel 1).
"""

import argparse
import json
import os
import re
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)

# Public datasheet figures, cross-checks only.
SPECS = {
    "gfx950": dict(name="MI355X", peak_tflops=2516.6, hbm_bytes_per_sec=8.0e12, cus=256, clock_hz=2.4e9,
                   mall_bytes=256 << 20),
}

BENCHMARKS = ["cal-mma", "cal-smem-bw", "cal-hbm-bw", "cal-latency"]


def detect_arch(text):
    m = re.search(r"GPU:.*\((gfx[0-9a-f]+)", text)
    return m.group(1) if m else None


def parse_results(text):
    """CAL_RESULT / CAL_INFO key-value lines, plus each column of the latency
    surface's saturation (CAL_SATURATION ilp <k> waves <w>) as
    warpsNeededToHideIlp<k>."""
    out = {}
    for line in text.splitlines():
        m = re.match(r"CAL_(?:RESULT|INFO)\s+(\S+)\s+(\S+)", line)
        if m:
            out[m.group(1)] = float(m.group(2))
            continue
        m = re.match(r"CAL_SATURATION\s+ilp\s+(\d+)\s+waves\s+(\d+)", line)
        if m:
            out["warpsNeededToHideIlp" + m.group(1)] = float(m.group(2))
    return out


def run_benchmark(binary_dir, name):
    path = os.path.join(binary_dir, name)
    if not os.path.exists(path):
        sys.exit("%s not found: build with `python -m ridge_amd.build`" % path)
    print("--- %s %s" % (name, "-" * (60 - len(name))), flush=True)
    proc = subprocess.run([path], capture_output=True, text=True)
    sys.stdout.write(proc.stdout)
    if proc.stderr:
        sys.stderr.write(proc.stderr)
    sys.stdout.flush()
    return parse_results(proc.stdout), proc.stdout, proc.returncode


def check(label, value, low, high, unit, note=""):
    ok = low <= value <= high
    print("  %-28s %12.4g %-12s band [%.4g, %.4g]  %s" % (label, value, unit, low, high,
                                                           "ok" if ok else "OUT OF BAND"))
    if note:
        print("  %-28s %s" % ("", note))
    return ok


def band_check(res, spec):
    """True when every constant sits in its sanity band."""
    ok = True
    ok &= check("impliedPeakTflopsNominal", res["impliedPeakTflopsNominalClock"], spec["peak_tflops"] * 0.85,
                spec["peak_tflops"] * 1.05, "TFLOP/s", "cycle count alone, at the nominal clock: tight band")
    ok &= check("clockHz", res["clockHz"] / 1e9, spec["clock_hz"] * 0.5 / 1e9, spec["clock_hz"] * 1.02 / 1e9,
                "GHz", "loaded clock; below nominal under power limits is expected")
    ok &= check("smemBytesPerCycle", res["smemBytesPerCycle"], 0.25 * res["ldsControlBytesPerCycle"],
                1.05 * res["ldsControlBytesPerCycle"], "B/cycle/CU", "bounded by the conflict-free control")
    ok &= check("hbmBytesPerSec", res["hbmBytesPerSec"] / 1e12, spec["hbm_bytes_per_sec"] * 0.60 / 1e12,
                spec["hbm_bytes_per_sec"] * 1.02 / 1e12, "TB/s", "above spec would mean the MALL, not HBM")
    if "hbmWriteBytesPerSec" in res:
        ok &= check("hbmWriteBytesPerSec", res["hbmWriteBytesPerSec"] / 1e12, spec["hbm_bytes_per_sec"] * 0.40 / 1e12,
                    spec["hbm_bytes_per_sec"] * 1.02 / 1e12, "TB/s", "streaming stores over 4 GiB")
    if "fillLatencySec" in res:
        ok &= check("fillLatencySec", res["fillLatencySec"] * 1e6, 0.2, 10.0, "us",
                    "first-tile wait of a whole grid from HBM")
    if "mallWriteBytesPerSec" in res and "hbmWriteBytesPerSec" in res:
        ok &= check("mallWriteBytesPerSec", res["mallWriteBytesPerSec"] / 1e12, 0.9 * res["hbmWriteBytesPerSec"] / 1e12,
                    4.0 * spec["hbm_bytes_per_sec"] / 1e12, "TB/s",
                    "cached stores into a MALL-resident buffer: not slower than to HBM")
    for i in (1, 2):
        key = "persistentStepCycles%d" % i
        if key in res and "pingPongMfmaCycles" in res:
            # Both persistent skeletons issue 32 MFMAs per SIMD per K tile, half
            # the ping-pong skeleton's K-step, and at best hide their reads.
            ok &= check(key, res[key], 0.45 * res["pingPongMfmaCycles"], 2.0 * res["pingPongMfmaCycles"], "cycles",
                        "persistent skeleton K tile: at least its MFMAs")
    for i in (1, 2):
        key = "pingPongRowStepCycles%d" % i
        if key in res and "pingPongMfmaCycles" in res:
            # Both row skeletons issue 64 MFMAs per SIMD per K tile, as the
            # ping-pong skeleton does; the schedule's waits and refill add to them.
            ok &= check(key, res[key], 0.9 * res["pingPongMfmaCycles"], 2.0 * res["pingPongMfmaCycles"], "cycles",
                        "ping-pong row skeleton K tile: at least its MFMAs")
    for i in (1, 2):
        key, step = "persistentTileCycles%d" % i, "persistentStepCycles%d" % i
        if key in res and step in res:
            # Staging one output tile through LDS and issuing its stores: not
            # negative, and a few K tiles at most.
            ok &= check(key, res[key], 0.0, 8.0 * res[step], "cycles",
                        "the epilogue between two output tiles of the persistent skeleton")
    if "mallRefillBytesPerSec" in res:
        ok &= check("mallRefillBytesPerSec", res["mallRefillBytesPerSec"] / 1e12, 1.0,
                    res["l2HitBytesPerCycle"] * res["clockHz"] / 1e12, "TB/s",
                    "L2-missing refill path: below what the L2s serve")
        ok &= check("mallStretch0", res["mallStretch0"], 0.95, 1.05, "x", "the all-hits skeleton against itself")
    if "launchOverheadSeconds" in res:
        ok &= check("launchSeconds", res["launchSeconds"] * 1e6, 0.5, 20.0, "us",
                    "back-to-back launches of a near-empty kernel")
        ok &= check("launchOverheadSeconds", res["launchOverheadSeconds"] * 1e6, 0.0, res["launchSeconds"] * 1e6,
                    "us", "kernel boundary on top of work, back to back: at most the empty-kernel floor")
        ok &= check("launchIsolatedSeconds", res["launchIsolatedSeconds"] * 1e6, res["launchOverheadSeconds"] * 1e6,
                    20.0, "us", "kernel boundary of one launch from an idle stream: at least the back-to-back one")
    ok &= check("warpsNeededToHide", res["warpsNeededToHide"], 1, 32, "waves/CU")
    # The L2s serve faster than HBM (at the loaded clock); 8 XCDs x 16 channels x
    # 128 B per cycle is the ceiling.
    ok &= check("l2HitBytesPerCycle", res["l2HitBytesPerCycle"], res["hbmBytesPerSec"] / res["clockHz"],
                8 * 16 * 128 * 1.05, "B/cycle", "above HBM at the loaded clock, below the L2 channels' peak")
    # A partly busy chip clocks at least as fast as a full one (within noise) and
    # never past the engine clock's ceiling.
    ceiling = spec["clock_hz"] * 1.05 / res["clockHz"]
    for key in CLOCK_RATIO_KEYS:
        ok &= check(key, res[key], 0.98, ceiling, "x", "over the full-chip loaded clock")
    ok &= check("freeRunningOverlap", res["freeRunningOverlap"], 0.0, 1.0, "",
                "share of the shorter phase two free-running waves per SIMD hide")
    ok &= check("loadedClockRatio", loaded_clock_ratio(res), 0.5, 1.0, "x",
                "skeleton clock with reads and refill over MFMAs alone; data movement costs power")
    ok &= check("ldsAReadBytesPerCycle", res["ldsAReadBytesPerCycle"], 0.25 * res["ldsControlBytesPerCycle"],
                1.05 * res["ldsControlBytesPerCycle"], "B/cycle/CU")
    ok &= check("ldsBTrReadBytesPerCycle", res["ldsBTrReadBytesPerCycle"], 0.125 * res["ldsControlBytesPerCycle"],
                1.05 * res["ldsControlBytesPerCycle"], "B/cycle/CU")
    return ok


CLOCK_RATIO_KEYS = ["clockRatioHalfCus", "clockRatioQuarterCus", "clockRatioEighthCus", "clockRatioSixteenthCus"]

# What the four benchmarks must report for a JSON to be written.
REQUIRED_KEYS = ["mmaCyclesPerInst", "impliedPeakTflops", "impliedPeakTflopsNominalClock", "clockHz",
                 "smemBytesPerCycle", "ldsControlBytesPerCycle", "ldsAReadBytesPerCycle", "ldsBTrReadBytesPerCycle",
                 "hbmBytesPerSec", "l2HitBytesPerCycle", "warpsNeededToHide", "pingPongMfmaCyclesClockHz",
                 "pingPongRefillStepCyclesClockHz", "freeRunningOverlap"] + CLOCK_RATIO_KEYS


def loaded_clock_ratio(res):
    """The ping-pong skeleton's clock with the GEMM's operand reads and refill over
    its clock with the MFMAs alone (cal-smem-bw): the model's powerModel 1."""
    return res["pingPongRefillStepCyclesClockHz"] / res["pingPongMfmaCyclesClockHz"]

# Figures of the ping-pong skeleton (cal-smem-bw), kept in the JSON as a record;
# the model reads none of them.
SKELETON_KEYS = ["pingPongStepCycles", "pingPongReadCycles", "pingPongMfmaCycles", "pingPongRefillStepCycles",
                 "pingPongStepCyclesClockHz", "pingPongMfmaCyclesClockHz", "pingPongRefillStepCyclesClockHz",
                 "phaseSwitchCycles"]


def hardware_json(res, spec, arch):
    out = {
        "name": spec["name"],
        "arch": arch,
        "note": ("measured by ridge_amd/calibrate.py on a %s; clockHz is the loaded clock measured by cal-mma "
                 "(clocks are not pinned on this machine); LDS rate is the GEMM's own read mix" % arch),
        "numSMs": spec["cus"],
        "clockHz": res["clockHz"],
        "mmaCyclesPerInst": res["mmaCyclesPerInst"],
        "smemBytesPerCycle": res["smemBytesPerCycle"],
        "hbmBytesPerSec": res["hbmBytesPerSec"],
        "regsPerSM": 131072,
        "smemBytesPerSM": 163840,
        "maxWarpsPerSM": 32,
        "maxCtasPerSM": 32,
        "warpsNeededToHide": res["warpsNeededToHide"],
        "waveSize": 64,
        "mmaM": 16,
        "mmaN": 16,
        "mmaK": 32,
        "simdsPerSM": 4,
        "regsPerSimdLane": 512,
        "regGranule": 8,
        "numXcds": 8,
        "cBytes": 2,
        "l2ReuseModel": 2,
        "prologueModel": 1,
        "pingPongModel": 1,
        "persistentModel": 1,
        "warpsNeededToHideIlp8": res.get("warpsNeededToHideIlp8", 0.0),
        "nominalClockHz": res.get("nominalClockHz", spec["clock_hz"]),
        "impliedPeakTflops": res["impliedPeakTflops"],
        "mallBytesPerSec": res.get("mallBytesPerSec", 0.0),
        "ldsControlBytesPerCycle": res["ldsControlBytesPerCycle"],
        "ldsAReadBytesPerCycle": res.get("ldsAReadBytesPerCycle", 0.0),
        "ldsBTrReadBytesPerCycle": res.get("ldsBTrReadBytesPerCycle", 0.0),
        "mfma32x32x16CyclesPerInst": res.get("mfma32x32x16CyclesPerInst", 0.0),
        "mfma32x32x16ClockHz": res.get("mfma32x32x16ClockHz", 0.0),
        "ldsReadModel": 1,
        "clockModel": 1,
        "l2StreamModel": 1,
        "l2HitBytesPerCycle": res["l2HitBytesPerCycle"],
        "uniformOverlapModel": 1,
        "freeRunningOverlap": res["freeRunningOverlap"],
        "powerModel": 1,
        "loadedClockRatio": loaded_clock_ratio(res),
        "fillShareModel": 1,
    }
    for key in CLOCK_RATIO_KEYS:
        out[key] = res[key]
    # Constants of the later calibration benches, written (with the model term
    # that reads them switched on) when the log has them.
    for key in (["hbmWriteBytesPerSec", "fillLatencySec", "mallRefillBytesPerSec", "persistentStepCycles1",
                 "persistentStepCycles2", "persistentTileCycles1", "persistentTileCycles2", "launchSeconds",
                 "launchOverheadSeconds", "launchIsolatedSeconds", "mallWriteBytesPerSec", "pingPongRowStepCycles1",
                 "pingPongRowStepCycles2"] +
                ["mallStretchLoad%d" % i for i in range(5)] + ["mallStretch%d" % i for i in range(5)]):
        if key in res:
            out[key] = res[key]
    if "mallRefillBytesPerSec" in res:
        # The MALL's capacity is a datasheet figure; the rate its hits move at
        # is the calibrated refill path's.
        out["mallBytes"] = spec["mall_bytes"]
        out["mallReuseModel"] = 1
    for term, needs in (("hbmWriteModel", ["hbmWriteBytesPerSec"]),
                        # No constant of its own: it overlaps the write stream with
                        # the L2-served loads (l2StreamModel is always on here).
                        ("writeOverlapModel", ["hbmWriteBytesPerSec"]),
                        ("fillLatencyModel", ["fillLatencySec"]),
                        ("mallStreamModel", ["mallRefillBytesPerSec"] + ["mallStretch%d" % i for i in range(5)]),
                        ("persistentStepModel", ["persistentStepCycles1", "persistentStepCycles2"]),
                        ("launchModel", ["launchOverheadSeconds"]),
                        ("mallWriteModel", ["mallWriteBytesPerSec", "hbmWriteBytesPerSec", "mallRefillBytesPerSec"]),
                        ("pingPongStepModel", ["pingPongRowStepCycles1", "pingPongRowStepCycles2"]),
                        ("labelModel", ["launchIsolatedSeconds", "hbmWriteBytesPerSec"])):
        if all(k in res for k in needs):
            out[term] = 1
    # persistentTileCycles1/2 (the epilogue between a persistent walk's tiles)
    # are written as a record; persistentTileModel, which reads them, stays off:
    # with the measured constants it raised MAPE and regret at k = 1 on the
    # in-sample sweep and on most held-out sweeps.
    if out.get("labelModel") == 1 and "nominalClockHz" in res:
        # The busy shares at the physical clock of the row's matrix load.
        out["labelModel"] = 2
    for key in SKELETON_KEYS:
        if key in res:
            out[key] = res[key]
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--binary-dir", default=os.path.join(PKG, "bin"))
    ap.add_argument("--out", default=os.path.join(ROOT, "data", "hardware", "mi355x.json"))
    ap.add_argument("--check", action="store_true", help="band-check only, write nothing")
    ap.add_argument("--log", default=None, help="also write the benchmarks' output here")
    ap.add_argument("--from-log", default=None,
                    help="derive the JSON from a saved benchmark log (a --log file) instead of running")
    args = ap.parse_args(argv)

    results, banner, failed = {}, "", False
    if args.from_log:
        with open(args.from_log) as f:
            banner = f.read()
        results = parse_results(banner)
    else:
        for name in BENCHMARKS:
            res, out, rc = run_benchmark(args.binary_dir, name)
            results.update(res)
            banner += out
            if rc != 0:
                print("  %s exited %d: its constants are unstable" % (name, rc))
                failed = True
            print()
    if args.log and not args.from_log:
        with open(args.log, "w") as f:
            f.write(banner)

    arch = detect_arch(banner)
    if arch is None:
        sys.exit("could not detect the GPU from the benchmark output")
    if arch not in SPECS:
        sys.exit("no datasheet entry for %s: add one to SPECS rather than reusing another card's" % arch)
    spec = SPECS[arch]
    missing = [k for k in REQUIRED_KEYS if k not in results]
    if missing:
        sys.exit("benchmarks did not report: %s" % ", ".join(missing))

    print("detected %s (%s); sanity bands against its datasheet:" % (spec["name"], arch))
    ok = band_check(results, spec)
    if failed:
        ok = False
        print("\n  at least one benchmark reported unstable repeats")
    print()
    if not ok:
        print("a constant is out of band or unstable: fix the benchmark rather than widening the band or "
              "importing a value from another GPU")
        return 1
    if args.check:
        print("all constants in band; run without --check to write")
        return 0
    os.makedirs(os.path.dirname(args.out) or ".", exist_ok=True)
    with open(args.out, "w") as f:
        json.dump(hardware_json(results, spec, arch), f, indent=2)
        f.write("\n")
    print("wrote", args.out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
