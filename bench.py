#!/usr/bin/env python3
"""Headline benchmark: FP16 GEMM TFLOP/s at 4096^3 on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--repeats R] [--variant BM,BN,BK,WM,WN,S,G]
                    [--shape M,N,K] [--split-tail BM,BN,BK,WM,WN,S,G [--split-rows R]]
                    [--no-cpu-baseline] [--no-blaslt] [--no-cold] [--no-autotune]
                    [--allow-partitioned]
    python bench.py --mode copy     # plain device copy of known size, for scaling
                                    # rocprofv3 FETCH_SIZE / WRITE_SIZE counters

A step is one C = A * B launch (FP16 A, B row-major from a seeded U[-1,1) device
fill, FP32 accumulate, FP16 C) through the C ABI, with inputs resident in HBM
before the timed region. 5 s of the same launches to bring the clock to its
loaded state, W untimed steps, then --repeats (default 5) windows of exactly K
steps, each bracketed by torch.cuda.synchronize(); value = 2 M N K K / elapsed of
the middle window, with the fastest and slowest windows in `spread`. The same
launches are also bracketed by HIP events on the launch stream for the roofline
figure. The hipBLASLt comparator (best of its heuristic candidates, best of a
before and an after reading, as the reference does in
bench/check-gemm.cu:357-391) and ours are compared on one basis: HIP events over
--repeats windows of max(K, 200) launches, warm and cold alike (hipBLASLt's host
time per call is close to one launch, and a short window would time the host).
Prints ONE JSON line.

cold: the same launches (ours and hipBLASLt's) rotated over enough operand sets
that twice the 256 MB MALL is touched between two uses of one set, so every
launch reads A and B from HBM; `value` is the warm figure (one operand set,
re-used, as the reference times). A device that is not a whole MI355X (gfx950,
256 CUs; a CPX/DPX partition is smaller) is refused unless --allow-partitioned.

cpu_baseline: the CPU f64 GEMM of the oracle (a port of the reference's CPU
reference, bench/check-gemm.cu:98-108, row-parallel with OpenMP) timed on a
bounded sample of the same 4096^3 workload (a block of output rows, about 10 s of
work), reported in TFLOP/s with the thread count used (the cores this process may
run on, at most 16).

model: the calibrated cost model's prediction for the measured variant and shape
(TFLOP/s, label, error against `value`), read from data/hardware/mi355x.json.

--split-tail: a step is a row split instead, two launches on one stream: --variant
on the first R rows of C (by default the rows of whole rounds of its resident
workgroups on this device's CUs, ridge_gemm_split_rows) and the tail row on the
remaining M - R. For grids whose last round of tiles would leave most CUs idle
(288 tiles of 256x256 on 256 CUs). `config.split` names both halves; the model
figure is the sum of the two predicted launch times; `roofline.traffic` is null
(no profile covers a pair of launches).

autotune: the metric's second half, the mean top-10 regret of the model-pruned
autotuner, is computed from the committed measured sweep of the current kernels
(data/measured/mi355x-current-kernels.csv, 14 shapes x 24 variants; the same sweep with
the previous kernels, data/measured/mi355x.csv, beside it) and the committed
calibration (data/hardware/mi355x.json)
by ridge_amd.autotune, with regret at top-1 and the expected regret of a random
shortlist beside it, and the same for the twelve held-out sweeps, each registered
before it was measured and scored with the constants frozen beside it
(data/measured/mi355x-heldout*.csv); it is a property of the sweeps and the model,
not of this run's timing.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# Datasheet dense FP16 MFMA peak of MI355X: 256 CUs x 4096 FLOP/clk/CU x 2.4 GHz.
PEAK_FP16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0
DEFAULT_SHAPE = (4096, 4096, 4096)
# The registered variant measured fastest at 4096^3 (the BASELINE-config
# measurement, data/measured/mi355x-baseline-configs.csv).
DEFAULT_VARIANT = (256, 256, 32, 128, 64, 3, 4)
PROFILES = os.path.join(ROOT, "profiles")
# The in-sample sweep measured with the current kernels, and the same sweep with
# the kernels before the steady K-loop passes (the set every earlier figure and
# the held-out comparisons refer to).
MEASURED_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-current-kernels.csv")
MEASURED_SWEEP_PREVIOUS = os.path.join(ROOT, "data", "measured", "mi355x.csv")
HARDWARE_JSON = os.path.join(ROOT, "data", "hardware", "mi355x.json")
HELDOUT_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout.csv")
HELDOUT_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout-hw.json")
HELDOUT2_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout2.csv")
HELDOUT2_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout2-hw.json")
HELDOUT3_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout3.csv")
HELDOUT3_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout3-hw.json")
HELDOUT4_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout4.csv")
HELDOUT4_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout4-hw.json")
HELDOUT5_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout5.csv")
HELDOUT5_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout5-hw.json")
HELDOUT6_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout6.csv")
HELDOUT6_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout6-hw.json")
HELDOUT7_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout7.csv")
HELDOUT7_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout7-hw.json")
HELDOUT8_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout8.csv")
HELDOUT8_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout8-hw.json")
HELDOUT9_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout9.csv")
HELDOUT9_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout9-hw.json")
HELDOUT10_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout10.csv")
HELDOUT10_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout10-hw.json")
HELDOUT11_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout11.csv")
HELDOUT11_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout11-hw.json")
HELDOUT12_SWEEP = os.path.join(ROOT, "data", "measured", "mi355x-heldout12.csv")
HELDOUT12_HARDWARE_JSON = os.path.join(ROOT, "data", "sweep", "mi355x-heldout12-hw.json")
# Host threads for the CPU baseline: the cores this process may use, capped at
# the 16 a GPU box grants one GPU.
MAX_CPU_THREADS = 16


def parse_ints(s, n):
    v = tuple(int(x) for x in s.split(","))
    if len(v) != n:
        raise SystemExit("expected %d comma-separated integers, got %r" % (n, s))
    return v


def time_launches(fn, steps, stream):
    """Wall time of `steps` calls bracketed by synchronize, and the HIP-event time
    of the same calls on the launch stream. Returns (wall_s, event_ms)."""
    import torch
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, e0.elapsed_time(e1)


def middle(xs):
    """Middle order statistic (mean of the two central values for an even count)."""
    ys = sorted(xs)
    h = len(ys) // 2
    return ys[h] if len(ys) % 2 else 0.5 * (ys[h - 1] + ys[h])


def time_windows(fn, steps, stream, repeats):
    """`repeats` windows of exactly `steps` launches each. Returns per-launch wall
    and HIP-event milliseconds, one entry per window, in the order timed."""
    wall_ms, event_ms = [], []
    for _ in range(repeats):
        wall, ev = time_launches(fn, steps, stream)
        wall_ms.append(wall * 1e3 / steps)
        event_ms.append(ev / steps)
    return wall_ms, event_ms


def window_summary(flops, per_launch_ms):
    """TFLOP/s of the middle window, with the fastest and slowest windows."""
    rates = [flops / (ms * 1e-3) / 1e12 for ms in per_launch_ms]
    mid = middle(rates)
    return {"tflops": round(mid, 3), "min": round(min(rates), 3), "max": round(max(rates), 3),
            "range_pct": round((max(rates) - min(rates)) / mid * 100, 2), "windows": len(rates)}


def calibrated_peaks():
    """The calibrated chip's own ceilings (data/hardware/mi355x.json): the MFMA
    rate a pure matrix load sustains at its loaded clock, and the HBM copy rate."""
    try:
        with open(HARDWARE_JSON) as f:
            hw = json.load(f)
        return float(hw["impliedPeakTflops"]), float(hw["hbmBytesPerSec"]) / 1e9
    except (OSError, KeyError, ValueError):
        return None, None


def roofline(M, N, K, per_launch_ms, traffic):
    """The bound the shape's arithmetic intensity puts it under (datasheet ridge
    point 2516.6 / 8 = 315 FLOP/B) and the algorithmic rate against it: FLOP/s for
    MFMA-bound shapes, compulsory bytes 2(MK + KN + MN) per second for HBM-bound
    ones, from the HIP-event time per launch. `peak` and `frac` are against the
    datasheet; `calibrated_peak` and `calibrated_frac` against the calibration."""
    flops = 2.0 * M * N * K
    nbytes = 2.0 * (M * K + K * N + M * N)
    sec = per_launch_ms * 1e-3
    cal_mfma, cal_hbm = calibrated_peaks()
    if flops / nbytes >= PEAK_FP16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9):
        achieved = flops / sec / 1e12
        out = {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
               "frac": round(achieved / PEAK_FP16_TFLOPS, 4), "traffic": traffic}
        cal = cal_mfma
    else:
        achieved = nbytes / sec / 1e9
        out = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
               "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic}
        cal = cal_hbm
    if cal:
        out["calibrated_peak"] = round(cal, 1)
        out["calibrated_frac"] = round(achieved / cal, 4)
    return out


# Infinity Cache (MALL) of MI355X: 256 MB, shared by all XCDs in front of HBM.
MALL_BYTES = 256 << 20
# Launches per window for the comparisons with hipBLASLt (warm and cold). Its
# calls go through ctypes and hipblasLtMatmul, whose host time per call is close
# to a 4096^3 launch; over a short window the GPU then waits on the host and the
# window times the host. Two hundred launches keep both queues ahead of the GPU.
COMPARE_LAUNCHES = 200
WHOLE_DEVICE_CUS = 256


def device_check(allow_partitioned):
    """Refuse anything but a whole MI355X (gfx950, 256 CUs): a compute-partitioned
    GPU (CPX, DPX) shows a fraction of the CUs and XCDs as its own device, which
    the sweep and the calibration do not describe (the reference refuses a MIG
    slice the same way, setup-box.sh:37-41). Returns the device description."""
    import torch
    p = torch.cuda.get_device_properties(0)
    arch = getattr(p, "gcnArchName", "")
    info = {"name": p.name, "arch": arch, "cus": p.multi_processor_count}
    if not (arch.startswith("gfx950") and p.multi_processor_count == WHOLE_DEVICE_CUS):
        msg = "device %s (%s, %d CUs) is not a whole MI355X (gfx950, %d CUs)" % (
            p.name, arch, p.multi_processor_count, WHOLE_DEVICE_CUS)
        if not allow_partitioned:
            raise SystemExit(msg + "; pass --allow-partitioned to run anyway")
        print(msg + "; continuing (--allow-partitioned)", file=sys.stderr)
    return info


def cold_sets(set_bytes):
    """Number of operand sets to rotate through so that at least twice the MALL's
    capacity of other sets is touched between two uses of one set."""
    return max(3, 1 + -(-2 * MALL_BYTES // set_bytes))


def time_cold(make_step, sets, steps, stream, repeats, warm_seconds):
    """HIP-event milliseconds per launch with launch i on operand set i % len(sets),
    so no launch finds its A, B or C in the MALL or the L2s; one entry per window
    of `steps` launches (the rotation continues across windows). The rotation
    first runs for `warm_seconds`: allocating and filling the extra sets leaves
    the GPU idle long enough for its clock to drop, and without this the first
    windows time the clock's ramp rather than the cold caches."""
    import torch
    n = len(sets)
    fns = [make_step(*s) for s in sets]
    t0 = time.perf_counter()
    while True:
        for f in fns:
            f()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= warm_seconds:
            break
    out = []
    j = 0
    for _ in range(repeats):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fns[j % n]()
            j += 1
        e1.record(stream)
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) / steps)
    return out


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, MAX_CPU_THREADS))


def measured_traffic(M, N, K, key, cold=False):
    """HBM bytes per launch from the committed rocprofv3 traffic summary for this
    shape and variant (its cold-rotation figure with cold=True), or None when no
    profile covers it."""
    if not os.path.isdir(PROFILES):
        return None
    for name in sorted(os.listdir(PROFILES)):
        if not name.endswith("_traffic.json"):
            continue
        with open(os.path.join(PROFILES, name)) as f:
            t = json.load(f)
        if tuple(t.get("shape", ())) == (M, N, K) and tuple(t.get("variant", ())) == key:
            return t.get("cold_hbm_bytes_per_launch" if cold else "hbm_bytes_per_launch")
    return None


def autotune_regret(k=10):
    """The pruner's regret at top-1 and top-k with the random-shortlist baseline,
    on the committed in-sample sweep measured with the current kernels
    (data/measured/mi355x-current-kernels.csv, 14 shapes x 24 variants, current
    calibration), on the same sweep with the previous kernels
    (data/measured/mi355x.csv) and on the twelve held-out sweeps, each
    registered before it was measured and scored with the constants frozen with
    it (data/measured/mi355x-heldout*.csv); a property of the
    sweeps and the model, not of this run's timing. None of it is computed if
    the model CLI is not built."""
    try:
        from ridge_amd import autotune as AT
        out = {"top_k": k, "source": os.path.relpath(MEASURED_SWEEP, ROOT)}
        for name, measured, hw in (("in_sample", MEASURED_SWEEP, HARDWARE_JSON),
                                   ("in_sample_previous_kernels", MEASURED_SWEEP_PREVIOUS, HARDWARE_JSON),
                                   ("held_out", HELDOUT_SWEEP, HELDOUT_HARDWARE_JSON),
                                   ("held_out_2", HELDOUT2_SWEEP, HELDOUT2_HARDWARE_JSON),
                                   ("held_out_3", HELDOUT3_SWEEP, HELDOUT3_HARDWARE_JSON),
                                   ("held_out_4", HELDOUT4_SWEEP, HELDOUT4_HARDWARE_JSON),
                                   ("held_out_5", HELDOUT5_SWEEP, HELDOUT5_HARDWARE_JSON),
                                   ("held_out_6", HELDOUT6_SWEEP, HELDOUT6_HARDWARE_JSON),
                                   ("held_out_7", HELDOUT7_SWEEP, HELDOUT7_HARDWARE_JSON),
                                   ("held_out_8", HELDOUT8_SWEEP, HELDOUT8_HARDWARE_JSON),
                                   ("held_out_9", HELDOUT9_SWEEP, HELDOUT9_HARDWARE_JSON),
                                   ("held_out_10", HELDOUT10_SWEEP, HELDOUT10_HARDWARE_JSON),
                                   ("held_out_11", HELDOUT11_SWEEP, HELDOUT11_HARDWARE_JSON),
                                   ("held_out_12", HELDOUT12_SWEEP, HELDOUT12_HARDWARE_JSON)):
            table, total, shapes, _ = AT.evaluate(measured, hw, ks=(1, k))
            base = AT.baselines(measured, hw, ks=(1, k))
            by_k = {r["k"]: r for r in table}
            entry = {"mean_regret_pct": round(by_k[k]["mean_regret"], 3),
                     "max_regret_pct": round(by_k[k]["max_regret"], 3), "exact_hits": by_k[k]["hits"],
                     "regret_at_1_mean_pct": round(by_k[1]["mean_regret"], 3),
                     "regret_at_1_max_pct": round(by_k[1]["max_regret"], 3),
                     "random_pick_at_1_pct": round(base[1]["random"][0], 3),
                     "random_pick_at_k_pct": round(base[k]["random"][0], 3),
                     "shapes": shapes, "configs": total,
                     "benchmarks_vs_exhaustive": round(by_k[k]["reduction"], 2),
                     "source": os.path.relpath(measured, ROOT)}
            if name == "in_sample":
                out.update({key: v for key, v in entry.items() if key != "source"})
            else:
                out[name] = entry
        return out
    except Exception as e:  # the model CLI is part of the build; report its absence
        return {"error": "%s" % e}


def model_prediction(v, M, N, K, measured):
    """The calibrated cost model's prediction for the variant this run measured:
    TFLOP/s, bottleneck label and the error against the measurement."""
    try:
        from ridge_amd import model as RM
        p = RM.predict(RM.Hardware(HARDWARE_JSON), M=M, N=N, K=K, BM=v.BM, BN=v.BN, BK=v.BK, warpM=v.WM,
                       warpN=v.WN, stages=v.stages, regsPerThread=v.regsPerThread, groupM=v.groupM,
                       schedule=v.schedule)
    except Exception as e:  # the model library is part of the build; report its absence
        return {"error": "%s" % e}
    return {"predicted_tflops": round(p["predictedTFLOPS"], 1), "label": p["bottleneck"],
            "error_pct": round((p["predictedTFLOPS"] - measured) / measured * 100, 1),
            "hardware": os.path.relpath(HARDWARE_JSON, ROOT)}


def model_split_prediction(body, tail, rows, M, N, K, measured):
    """The cost model's figure for a row split: the predicted times of the body
    launch (rows x N x K) and the tail launch ((M - rows) x N x K), added, since
    the two run one after the other on one stream."""
    try:
        from ridge_amd import model as RM
        hw = RM.Hardware(HARDWARE_JSON)
        secs, labels = 0.0, []
        for v, m in ((body, rows), (tail, M - rows)):
            p = RM.predict(hw, M=m, N=N, K=K, BM=v.BM, BN=v.BN, BK=v.BK, warpM=v.WM, warpN=v.WN,
                           stages=v.stages, regsPerThread=v.regsPerThread, groupM=v.groupM, schedule=v.schedule)
            secs += 2.0 * m * N * K / (p["predictedTFLOPS"] * 1e12)
            labels.append(p["bottleneck"])
    except Exception as e:  # the model library is part of the build; report its absence
        return {"error": "%s" % e}
    tflops = 2.0 * M * N * K / secs / 1e12
    return {"predicted_tflops": round(tflops, 1), "label": "+".join(labels),
            "error_pct": round((tflops - measured) / measured * 100, 1),
            "hardware": os.path.relpath(HARDWARE_JSON, ROOT)}


def cpu_baseline(M, N, K, seconds=10.0):
    """f64 oracle GEMM on a block of output rows of the same workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as O
    Ab = O.uniform_fill_f16(M * K, 1).reshape(M, K)
    Bb = O.uniform_fill_f16(K * N, 2)
    threads = cpu_threads()
    # Grow the row block until one call takes about `seconds` (each call also
    # pays the one-off conversion of B, which the first small blocks are
    # dominated by, so the estimate is refined from the previous call).
    rows = 16
    while True:
        t0 = time.perf_counter()
        O.gemm_f64(Ab[:rows].ravel(), Bb, rows, N, K, threads=threads)
        dt = time.perf_counter() - t0
        if dt >= 0.5 * seconds or rows >= M:
            break
        rows = int(min(M, max(2 * rows, rows * seconds / max(dt, 1e-3))))
    tflops = 2.0 * rows * N * K / dt / 1e12
    return {"value": round(tflops, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": "%d of %d output rows of %dx%dx%d (f64 accumulate, %.1f s)" % (rows, M, M, N, K, dt)}


def cpu_baseline_naive_1core(n=1024, seconds=2.0):
    """The reference's own CPU path, faithfully: the naive single-threaded i-j-k
    f64 loop (check-gemm.cu:98-108) at 1024^3, where the reference uses it, on a
    block of output rows."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    Ab = O.uniform_fill_f16(n * n, 1).reshape(n, n)
    Bb = O.uniform_fill_f16(n * n, 2)
    rows = 4
    while True:
        t0 = time.perf_counter()
        O.gemm_f64(Ab[:rows].ravel(), Bb, rows, n, n, naive=True)
        dt = time.perf_counter() - t0
        if dt >= 0.5 * seconds or rows >= n:
            break
        rows = int(min(n, max(2 * rows, rows * seconds / max(dt, 1e-4))))
    return {"value": round(2.0 * rows * n * n / dt / 1e12, 9), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": "%d of %d output rows of %d^3, naive i-j-k f64 loop (%.2f s)" % (rows, n, n, dt)}


def run_copy_mode(steps):
    """A plain device-to-device copy of known size, the scaling reference for the
    rocprofv3 FETCH_SIZE and WRITE_SIZE counters."""
    import torch
    nbytes = 256 << 20
    src = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda:0")
    dst = torch.empty_like(src)
    src.fill_(1.0)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "copy", "bytes_per_copy": nbytes, "copies": steps}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--variant", default=",".join(str(x) for x in DEFAULT_VARIANT))
    ap.add_argument("--shape", default=",".join(str(x) for x in DEFAULT_SHAPE))
    ap.add_argument("--warm-seconds", type=float, default=5.0)
    ap.add_argument("--cold-warm-seconds", type=float, default=2.0,
                    help="seconds the cold rotation runs before its windows are timed (capped by --warm-seconds)")
    ap.add_argument("--repeats", type=int, default=5,
                    help="timed windows of --steps launches each; figures are the middle window")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-blaslt", action="store_true")
    ap.add_argument("--no-cold", action="store_true")
    ap.add_argument("--allow-partitioned", action="store_true")
    ap.add_argument("--mode", default="gemm", choices=["gemm", "copy"])
    ap.add_argument("--split-tail", default=None,
                    help="tail row BM,BN,BK,WM,WN,S,G of a row split; --variant runs the body rows")
    ap.add_argument("--split-rows", type=int, default=None,
                    help="body rows of the split (default: whole rounds of --variant's workgroups)")
    ap.add_argument("--no-autotune", action="store_true",
                    help="leave out the autotune regret object (a property of the committed sweeps)")
    args = ap.parse_args()

    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the GEMM is "
              "single-device by design; see the sharding notes). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    if args.mode == "copy":
        run_copy_mode(max(args.steps, 1))
        return
    device = device_check(args.allow_partitioned)

    from ridge_amd import gemm as G

    M, N, K = parse_ints(args.shape, 3)
    key = parse_ints(args.variant, 7)
    idx = G.find_variant(*key)
    if idx < 0:
        raise SystemExit("variant %s is not in the registered table" % (key,))
    v = G.variant(idx)
    split = None
    if args.split_tail is not None:
        tidx = G.find_variant(*parse_ints(args.split_tail, 7))
        if tidx < 0:
            raise SystemExit("split tail %s is not in the registered table" % (args.split_tail,))
        rows = args.split_rows
        if rows is None:
            rows = G.split_rows(idx, M, N, K, device["cus"])
            if rows <= 0 or rows >= M:
                why = ("the row does not divide the shape" if rows < 0 else
                       "the grid is under one round of resident workgroups" if rows == 0 else
                       "the grid is a whole number of rounds")
                raise SystemExit("no row split of %dx%dx%d for %s on %d CUs: %s"
                                 % (M, N, K, v.label(), device["cus"], why))
        tv = G.variant(tidx)
        if not (0 < rows < M and v.divides(rows, N, K) and tv.divides(M - rows, N, K)):
            raise SystemExit("split of %dx%dx%d at %d rows: %s must divide the body and %s the tail"
                             % (M, N, K, rows, v.label(), tv.label()))
        split = (tidx, tv, rows)
    elif not v.divides(M, N, K):
        raise SystemExit("variant %s does not divide %dx%dx%d" % (v.label(), M, N, K))

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    A = torch.empty((M, K), dtype=torch.float16, device=dev)
    B = torch.empty((K, N), dtype=torch.float16, device=dev)
    C = torch.empty((M, N), dtype=torch.float16, device=dev)
    def fill(a, b):
        G.fill_uniform(a, 1)
        G.fill_uniform(b, 2)

    fill(A, B)
    torch.cuda.synchronize()
    flops = 2.0 * M * N * K

    # Both kernels are called through one foreign call with pre-converted
    # arguments, so neither side's host cost reaches a window (at 1024^3 a launch
    # is 6 us, about what converting the tensor arguments costs in Python).
    def make_step(a, b, c):
        if split is None:
            return G.bound_launch(idx, a, b, c, M, N, K, stream)
        return G.bound_launch_split(idx, split[0], split[2], a, b, c, M, N, K, stream)

    step = make_step(A, B, C)

    # Clock ramp: seconds of the same work before anything is timed (the
    # reference warms 5 s, check-gemm.cu:41-45).
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < args.warm_seconds:
        for _ in range(50):
            step()
        torch.cuda.synchronize()
    repeats = max(1, args.repeats)
    compare_steps = max(args.steps, COMPARE_LAUNCHES)

    blas = None
    blas_before = blas_after = None
    blas_error = None
    if not args.no_blaslt:
        # The comparator is context, not the measurement: if hipBLASLt cannot
        # serve the shape, the line still reports `value` and says why.
        try:
            blas = G.BlasLt()
            blas.prepare(A, B, C, M, N, K, candidates=16, iters=20, stream=stream)
        except G.RidgeGemmError as e:
            blas, blas_error = None, str(e)
    if blas is not None:
        blas_step = blas.bound_gemm(A, B, C, M, N, K, stream=stream)
        for _ in range(args.warmup):
            blas_step()
        _, blas_before = time_windows(blas_step, compare_steps, stream, repeats)

    # The timed region proper: W untimed steps, then `repeats` windows of exactly
    # K steps, each bracketed by torch.cuda.synchronize(); `value` is the middle
    # window's wall-clock rate.
    for _ in range(args.warmup):
        step()
    wall_ms, event_ms = time_windows(step, args.steps, stream, repeats)
    mid_wall_ms = middle(wall_ms)
    value = flops / (mid_wall_ms * 1e-3) / 1e12
    per_launch_ms = middle(event_ms)

    if blas is not None:
        # Ours on the comparison's own basis (HIP events, windows of
        # compare_steps launches), between hipBLASLt's two readings.
        _, ours_compare = time_windows(step, compare_steps, stream, repeats)
        _, blas_after = time_windows(blas_step, compare_steps, stream, repeats)
        blas.close()

    # Cold: the same launches rotated over operand sets that together exceed
    # twice the MALL, so every launch streams A and B from HBM (and writes C to
    # lines no cache holds). The warm figure above re-uses one set, as the
    # reference's timing loop does (measure.cu:111-150).
    cold = None
    if not args.no_cold:
        set_bytes = 2 * (M * K + K * N + M * N)
        n_sets = cold_sets(set_bytes)
        sets = [(A, B, C)]
        for i in range(1, n_sets):
            Ai = torch.empty_like(A)
            Bi = torch.empty_like(B)
            fill(Ai, Bi)
            sets.append((Ai, Bi, torch.empty_like(C)))
        torch.cuda.synchronize()
        cold_steps = max(args.steps // 4, 4 * n_sets, COMPARE_LAUNCHES // 2)
        cold_warm_s = max(0.0, min(args.cold_warm_seconds, args.warm_seconds))
        cold_windows = time_cold(make_step, sets, cold_steps, stream, repeats, cold_warm_s)
        cold_ms = middle(cold_windows)
        cold = {"tflops": round(flops / (cold_ms * 1e-3) / 1e12, 3), "ms_per_launch": round(cold_ms, 6),
                "spread": window_summary(flops, cold_windows),
                "sets": n_sets, "set_bytes": set_bytes, "launches_per_window": cold_steps,
                "rotation_warm_seconds": cold_warm_s,
                "roofline": roofline(M, N, K, cold_ms,
                                     None if split else measured_traffic(M, N, K, key, cold=True))}
        if blas is not None:
            try:
                blas = G.BlasLt()
                blas.prepare(A, B, C, M, N, K, candidates=16, iters=20, stream=stream)
            except G.RidgeGemmError as e:
                blas = None
                cold["hipblaslt_error"] = str(e)
        if blas is not None:

            def make_blas_step(a, b, c):
                return blas.bound_gemm(a, b, c, M, N, K, stream=stream)

            blas_cold_ms = middle(time_cold(make_blas_step, sets, cold_steps, stream, repeats, cold_warm_s))
            blas.close()
            cold["hipblaslt_tflops"] = round(flops / (blas_cold_ms * 1e-3) / 1e12, 3)
            cold["frac_of_hipblaslt"] = round(blas_cold_ms / cold_ms, 4)
        del sets

    traffic = None if split else measured_traffic(M, N, K, key)

    out = {
        "metric": "FP16 GEMM TFLOP/s @4096^3 on 1 MI355X (% MFMA peak, % hipBLASLt); top-10 regret"
                  if (M, N, K) == DEFAULT_SHAPE else "FP16 GEMM TFLOP/s @%dx%dx%d on 1 MI355X" % (M, N, K),
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mid_wall_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: A, B ~ U[-1,1) FP16 from splitmix64 seeds 1 and 2, generated on the device",
        "config": {"workload": "FP16 GEMM M=%d N=%d K=%d, row-major A/B/C, FP32 accumulate, FP16 C" % (M, N, K),
                   "variant": v.label(), "parallelism": "single GPU"},
        "repeats": repeats,
        "spread": window_summary(flops, wall_ms),
        "warm_seconds": args.warm_seconds,
        "frac_of_mfma_peak": round(value / PEAK_FP16_TFLOPS, 4),
        "roofline": roofline(M, N, K, per_launch_ms, traffic),
    }
    if blas_error is not None:
        out["hipblaslt"] = {"error": blas_error}
    if blas_before is not None:
        # Both sides on one basis: HIP events over windows of compare_steps
        # launches, middle window; hipBLASLt is the better of its readings
        # before and after ours (bench/check-gemm.cu:357-391).
        before = flops / (middle(blas_before) * 1e-3) / 1e12
        after = flops / (middle(blas_after) * 1e-3) / 1e12
        best = max(before, after)
        ours = flops / (middle(ours_compare) * 1e-3) / 1e12
        out["hipblaslt"] = {"tflops": round(best, 3), "before": round(before, 3), "after": round(after, 3),
                            "drift": round(abs(after - before) / before, 4),
                            "spread": window_summary(flops, blas_before if before >= after else blas_after),
                            "ours_tflops": round(ours, 3),
                            "basis": "HIP events, %d windows of %d launches, middle window" % (repeats, compare_steps),
                            "frac_of_hipblaslt": round(ours / best, 4)}
    if split is not None:
        out["config"]["split"] = {"body_rows": split[2], "tail": split[1].label(), "tail_rows": M - split[2],
                                  "body_rows_planned": args.split_rows is None}
    if cold is not None:
        out["cold"] = cold
    out["device"] = device
    if not args.no_autotune:
        out["autotune"] = autotune_regret(10)
    if split is None:
        out["model"] = model_prediction(v, M, N, K, value)
    else:
        out["model"] = model_split_prediction(v, split[1], split[2], M, N, K, value)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(M, N, K)
        out["cpu_baseline_naive_1core"] = cpu_baseline_naive_1core()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
