"""Cross-check of the cost model's bottleneck labels against rocprofv3 counters:
the MI355X restatement of the reference's bench/run-ncu-validation.sh and its
pre-registered decision tables (data/sweep/ncu-label-mapping.md).

    python -m ridge_amd.labelcheck [--registration N] select   # the registered config list
    python -m ridge_amd.labelcheck [--registration N] run      # the launches, under rocprofv3
    python -m ridge_amd.labelcheck [--registration N] gather --counters D1 --fetch D2 --write D3 --trace D4
    python -m ridge_amd.labelcheck [--registration N] score    # the registered decision table

Each registration fixes, in files committed before its first run, the decision
table, the counters, the config-selection rule, the pass criterion and a frozen
copy of the calibration and of the measured rows the selection was made from:
  1  data/sweep/rocprof-label-mapping.md (scored 5 of 13: FAIL; stands as is)
  2  data/sweep/rocprof-label2-mapping.md (the current kernel table and model;
     ENVELOPE decided from durations at K and 16 K, HBM% against the calibrated
     read and write rates, no fall-through label)
`run` and `gather` only launch kernels and collect numbers; `score` applies the
registered table and nothing else, so the rule cannot drift after the data
exists (the reference's own discipline, run-ncu-validation.sh:1-6).

`run` must be the program rocprofv3 starts (`rocprofv3 ... -- python3 -m
ridge_amd.labelcheck run`). It launches, for every config in order, the
registered variant LAUNCHES times on seeded U[-1,1) inputs (and, for a
registration with a long factor F, LAUNCHES more times at K x F); `gather`
assigns the GEMM dispatches of each rocprofv3 pass to configs by dispatch order
and checks every dispatch's kernel name against the config's template arguments.
"""

import argparse
import csv
import glob
import json
import os
import re
import statistics
import sys

from ridge_amd import model as RM
from ridge_amd.rocprof import counter_value, parse_counter_dir, parse_trace_dir  # noqa: F401
from ridge_amd import tables as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SWEEP_DIR = os.path.join(ROOT, "data", "sweep")


class Registration:
    """The files of one registration. `hw_json` is a frozen copy of
    data/hardware/mi355x.json at registration time and `sources` frozen copies
    of the measured rows the selection was made from, so a later re-calibration
    or re-measurement cannot change the registered configs or thresholds.
    `factors(config)` lists the K multipliers every config is launched at
    (LAUNCHES launches each, the multiplier 1 first): registration 2 adds K x 16
    (`long_factor`), the design set K / 2 (where BK divides it) and K x 2."""

    def __init__(self, number, stem, long_factor=0, factors=None):
        self.number = number
        self.stem = stem
        self.mapping = os.path.join(SWEEP_DIR, stem + "-mapping.md")
        self.hw_json = os.path.join(SWEEP_DIR, stem + "-hw.json")
        self.sources = [os.path.join(SWEEP_DIR, stem + "-sweep.csv"),
                        os.path.join(SWEEP_DIR, stem + "-baseline-configs.csv")]
        self.configs = os.path.join(SWEEP_DIR, stem + "-configs.csv")
        self.counters = os.path.join(ROOT, "data", "measured", stem.replace("rocprof-label", "rocprof-labels") + ".csv")
        self.long_factor = long_factor
        self._factors = factors

    def factors(self, c):
        if self._factors is not None:
            return self._factors(c)
        return [1, self.long_factor] if self.long_factor else [1]

    def duration_column(self, f):
        if f == 1:
            return "duration_ns"
        if f == self.long_factor:
            return "long_duration_ns"
        return "duration_x%g_ns" % f


def design_factors(c):
    """K / 2 where it is a whole number of K tiles, and K x 2."""
    half = c["K"] // 2
    return [1] + ([0.5] if c["K"] % 2 == 0 and half % c["BK"] == 0 and half >= c["BK"] else []) + [2]


def body_factors(c):
    """Registration 3: the second K of the body share, K / 2 when that is a whole
    number of K tiles (at least one), else K x 2; the model's labelModel 1 uses
    the same rule (Prediction.bodyFactor)."""
    half = c["K"] // 2
    return [1, 0.5] if c["K"] % 2 == 0 and half % c["BK"] == 0 and half >= c["BK"] else [1, 2]


REGISTRATIONS = {1: Registration(1, "rocprof-label", 0), 2: Registration(2, "rocprof-label2", 16),
                 3: Registration(3, "rocprof-label3", factors=body_factors),
                 4: Registration(4, "rocprof-label4", factors=body_factors),
                 "design": Registration("design", "rocprof-label-design", factors=design_factors)}
CURRENT = 4
# Registrations 3 and 4 share the decision table; each draws its fresh configs
# from the cross product of a held-out sweep registered with it.
REGISTRATIONS[3].heldout_shapes = os.path.join(SWEEP_DIR, "mi355x-heldout5-registered.csv")
REGISTRATIONS[4].heldout_shapes = os.path.join(SWEEP_DIR, "mi355x-heldout6-registered.csv")
for _r in (REGISTRATIONS[3], REGISTRATIONS[4]):
    _r.table = os.path.join(SWEEP_DIR, _r.stem + "-table.csv")
TABLE_RULE_REGISTRATIONS = (3, 4)
# Registration 1's files under their original names (kept for its tests).
HW_JSON = REGISTRATIONS[1].hw_json
SOURCES = REGISTRATIONS[1].sources
CONFIGS_CSV = REGISTRATIONS[1].configs
COUNTERS_CSV = REGISTRATIONS[1].counters

LAUNCHES = 3
PER_LABEL = 4
LABEL_ORDER = ["SMEM", "WAVES", "ENVELOPE", "OCC", "HBM", "TENSOR_CORE"]

# Registered decision table (data/sweep/rocprof-label-mapping.md section 2),
# applied top to bottom, first match wins.
HBM_PCT_MIN = 70.0          # rule 1: HBM% >= 70            -> HBM
SIMD_UTIL_PCT_MAX = 80.0    # rule 2: SIMD utilisation < 80 -> WAVES
OCC_SHORTFALL_MAX = 0.70    # rule 3: achieved/theoretical waves < 0.70 -> OCC
MFMA_PCT_MIN = 70.0         # rule 5: MFMA% >= 70           -> TENSOR_CORE
PASS_FRACTION = 0.75        # pass: at least 75% of configs agree

# Traffic scaling of FETCH_SIZE / WRITE_SIZE on this chip: a 256 MiB device
# copy reads FETCH_SIZE 131,083.5 KiB and WRITE_SIZE 262,144 KiB.
FETCH_SCALE = 2.000
WRITE_SCALE = 1.000

PASS1_COUNTERS = ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES", "SQ_WAVE_CYCLES", "SQ_LDS_IDX_ACTIVE",
                  "SQ_WAVES", "SQ_INSTS_MFMA", "GRBM_GUI_ACTIVE", "GRBM_COUNT"]

KEY_FIELDS = ["BM", "BN", "BK", "WM", "WN", "stages", "groupM"]
# 4096^3 with the bench's default variant at registration time.
CONTROL = (4096, 4096, 4096, 256, 256, 32, 128, 64, 4, 4)
CONTROL_SIMD_UTIL_PCT = (80.0, 105.0)


def _read_rows(path):
    return T.read(path).records


def predict_row(hw, r, with_schedule=False):
    """The model on a measured row. Registration 2 passes the row's schedule (the
    persistent rows are modelled as such); registration 1 did not, and keeps
    selecting as it did."""
    extra = {"schedule": int(r["schedule"])} if with_schedule and "schedule" in r else {}
    return RM.predict(hw, M=int(r["M"]), N=int(r["N"]), K=int(r["K"]), BM=int(r["BM"]), BN=int(r["BN"]),
                      BK=int(r["BK"]), warpM=int(r["WM"]), warpN=int(r["WN"]), stages=int(r["stages"]),
                      regsPerThread=int(r["regsPerThread"]), groupM=int(r["groupM"]), **extra)


def _config_row(label, r, p, why=None):
    row = {"predicted_label": label, "model_label": p["bottleneck"], "tag": r["tag"], "M": int(r["M"]),
           "N": int(r["N"]), "K": int(r["K"]), **{k: int(r[k]) for k in KEY_FIELDS},
           "regsPerThread": int(r["regsPerThread"]), "theoretical_waves_per_cu": p["ctasPerSM"] * p["numWarps"],
           "pred_tflops": round(p["predictedTFLOPS"], 3), "measured_tflops": float(r["tflops"])}
    if why is not None:
        row["schedule"] = int(r["schedule"])
        row["why"] = why
    return row


def _key(r):
    return tuple(int(r[k]) for k in ["M", "N", "K"] + KEY_FIELDS)


# Registration 2's required configs, scored beside the per-label selection:
# (shape + tile key, reason). The headline row also serves as the control.
REQUIRED_2 = [
    ((4096, 4096, 4096, 256, 256, 32, 128, 64, 3, 4), "headline ping-pong row"),
    ((4096, 4096, 4096, 256, 128, 64, 64, 64, 3, 8), "8-wave ping-pong row, 256x128 tile"),
    ((8192, 8192, 128, 128, 128, 64, 64, 64, 4, 8), "persistent row, K = 128"),
    ((8192, 8192, 128, 256, 128, 32, 64, 64, 6, 4), "persistent row, K = 128"),
    ((16384, 128, 8192, 128, 64, 64, 64, 32, 6, 8), "persistent row, tall-skinny"),
]
CONTROL_2 = REQUIRED_2[0][0]

# Registration 3 (data/sweep/rocprof-label3-mapping.md): configs drawn from the
# fifth held-out sweep's cross product (registered, not yet measured) plus the
# BASELINE configs' best rows.
HELDOUT5_SHAPES = os.path.join(SWEEP_DIR, "mi355x-heldout5-registered.csv")
TABLE3 = os.path.join(SWEEP_DIR, "rocprof-label3-table.csv")
LABEL_ORDER_3 = ["HBM", "WAVES", "ENVELOPE", "SMEM", "TENSOR_CORE", "OCC"]
REQUIRED_3 = [
    ((4096, 4096, 4096, 256, 256, 32, 128, 64, 3, 4), "baseline-4096cube-headline", "control: the headline row"),
    ((1024, 1024, 1024, 64, 64, 64, 32, 32, 4, 8), "baseline-1024cube", "required: BASELINE config, best row"),
    ((8192, 8192, 128, 256, 128, 32, 64, 64, 6, 4), "baseline-small-k", "required: BASELINE config, best row"),
    ((16384, 128, 8192, 64, 128, 128, 32, 64, 3, 8), "baseline-tall-skinny", "required: BASELINE config, best row"),
]
TABLE3_COLUMNS = KEY_FIELDS + ["persistent", "regsPerThread", "schedule"]


def write_table3(path=TABLE3):
    """The kernel table at registration time with each row's register count and
    schedule (from the built library), so the selection re-derives without it."""
    from ridge_amd import gemm as G
    rows = [dict(BM=v.BM, BN=v.BN, BK=v.BK, WM=v.WM, WN=v.WN, stages=v.stages, groupM=v.groupM,
                 persistent=int(v.schedule == 2), regsPerThread=v.regsPerThread, schedule=v.schedule)
            for v in G.variants()]
    T.write(path, TABLE3_COLUMNS, rows, ["the kernel table registration 3 is selected from (ridge_amd/csrc/"
                                         "gemm_variants.def and the compiler's register counts at registration)"])


def select_configs3(reg):
    """Registration 3's rule. Every shape of the fifth held-out sweep times every
    row of the frozen table is labelled by the frozen model; within each label
    (in LABEL_ORDER_3) the configs are sorted by (tag, BM, BN, BK, WM, WN, stages,
    groupM) and the first PER_LABEL of distinct shapes are taken. The control and
    the BASELINE configs' best rows (REQUIRED_3) come first."""
    hw = RM.Hardware(reg.hw_json)
    table = [{k: int(v) for k, v in r.items()} for r in _read_rows(reg.table)]
    by_key = {tuple(t[k] for k in KEY_FIELDS): t for t in table}

    def config(M, N, K, t, tag):
        r = {"M": M, "N": N, "K": K, "tag": tag, "regsPerThread": t["regsPerThread"], "schedule": t["schedule"],
             **{k: t[k] for k in KEY_FIELDS}}
        p = predict_row(hw, r, True)
        return r, p

    def row(label, r, p, why):
        return {"predicted_label": label, "model_label": p["bottleneck"], "tag": r["tag"], "M": r["M"], "N": r["N"],
                "K": r["K"], **{k: r[k] for k in KEY_FIELDS}, "regsPerThread": r["regsPerThread"],
                "theoretical_waves_per_cu": p["ctasPerSM"] * p["numWarps"],
                "pred_tflops": round(p["predictedTFLOPS"], 3), "measured_tflops": "", "schedule": r["schedule"],
                "why": why}

    out = []
    for key, tag, why in REQUIRED_3:
        r, p = config(key[0], key[1], key[2], by_key[key[3:]], tag)
        out.append(row("CONTROL" if why.startswith("control") else p["bottleneck"], r, p, why))
    groups = {}
    for M, N, K, tag in T.read_shapes(reg.heldout_shapes):
        for t in table:
            r, p = config(M, N, K, t, tag)
            groups.setdefault(p["bottleneck"], []).append((r, p))
    for label in LABEL_ORDER_3:
        shapes = set()
        for r, p in sorted(groups.get(label, []), key=lambda rp: (rp[0]["tag"],) + tuple(rp[0][k] for k in KEY_FIELDS)):
            shape = (r["M"], r["N"], r["K"])
            if shape in shapes:
                continue
            shapes.add(shape)
            out.append(row(label, r, p, "per-label rule"))
            if len(shapes) == PER_LABEL:
                break
    return out


def select_configs(sources=SOURCES, hw_json=HW_JSON, per_label=PER_LABEL, registration=1):
    """The registered selection rule: every measured row (sweep and BASELINE
    configs) is labelled by the model; within each label the rows are sorted by
    (tag, BM, BN, BK, WM, WN, stages, groupM) and the first `per_label` rows of
    distinct shapes are taken (the reference's rule, ncu-label-mapping.md
    section 3). Registration 2 labels with each row's schedule and adds the
    configs of REQUIRED_2 that the rule did not pick."""
    second = registration == 2
    hw = RM.Hardware(hw_json)
    groups, by_key = {}, {}
    for src in sources:
        for r in _read_rows(src):
            p = predict_row(hw, r, second)
            groups.setdefault(p["bottleneck"], []).append((r, p))
            by_key.setdefault(_key(r), (r, p))
    out = []
    # The control: one workgroup per CU for the whole launch keeps every CU busy,
    # which checks the counter normalisations (section 2 of each registration).
    control = CONTROL_2 if second else CONTROL
    for r in _read_rows(sources[-1]):
        if _key(r) == control:
            p = predict_row(hw, r, second)
            out.append(_config_row("CONTROL", r, p, "control" if second else None))
    picked = set()
    for label in LABEL_ORDER:
        rows = sorted(groups.get(label, []),
                      key=lambda rp: (rp[0]["tag"],) + tuple(int(rp[0][k]) for k in KEY_FIELDS))
        shapes = set()
        for r, p in rows:
            shape = (int(r["M"]), int(r["N"]), int(r["K"]))
            if shape in shapes:
                continue
            shapes.add(shape)
            picked.add(_key(r))
            out.append(_config_row(label, r, p, "per-label rule" if second else None))
            if len(shapes) == per_label:
                break
    if second:
        for key, why in REQUIRED_2:
            if key in picked:
                continue
            r, p = by_key[key]
            out.append(_config_row(p["bottleneck"], r, p, "required: " + why))
    return out


def design_configs():
    """The label-design set: in-sample rows the decision rules and the model's
    counter predictions are developed on, never scored. Every config of
    registrations 1 and 2 whose variant is still in the kernel table; for each
    of the 14 in-sample sweep shapes (data/measured/mi355x.csv) its fastest,
    median and slowest measured row; and the fastest row of each BASELINE config
    (data/measured/mi355x-baseline-configs.csv). Configs are keyed by shape and
    tile; the first occurrence is kept."""
    from ridge_amd import validate as V
    table = set(V.kernel_table_keys())
    hw = RM.Hardware(os.path.join(ROOT, "data", "hardware", "mi355x.json"))
    measured = {}
    for name in ("mi355x.csv", "mi355x-baseline-configs.csv"):
        for r in _read_rows(os.path.join(ROOT, "data", "measured", name)):
            measured.setdefault(_key(r), r)
    out, seen = [], set()

    def add(r, why):
        key = _key(r)
        if key in seen or tuple(int(r[k]) for k in KEY_FIELDS) not in table:
            return
        seen.add(key)
        m = measured.get(key, r)
        row = dict(m)
        p = predict_row(hw, row, True)
        out.append(_config_row("DESIGN", row, p, why))

    for reg in (1, 2):
        for c in _read_rows(REGISTRATIONS[reg].configs):
            key = _key(c)
            if key in measured:
                add(measured[key], "registration %d config" % reg)
    sweep = _read_rows(os.path.join(ROOT, "data", "measured", "mi355x.csv"))
    for shape in sorted({(int(r["M"]), int(r["N"]), int(r["K"])) for r in sweep}):
        rows = sorted((r for r in sweep if (int(r["M"]), int(r["N"]), int(r["K"])) == shape),
                      key=lambda r: (-float(r["tflops"]),) + tuple(int(r[k]) for k in KEY_FIELDS))
        for pos, why in ((0, "fastest"), (len(rows) // 2, "median"), (len(rows) - 1, "slowest")):
            add(rows[pos], "in-sample shape, %s row" % why)
    base = _read_rows(os.path.join(ROOT, "data", "measured", "mi355x-baseline-configs.csv"))
    for shape in sorted({(int(r["M"]), int(r["N"]), int(r["K"])) for r in base}):
        rows = [r for r in base if (int(r["M"]), int(r["N"]), int(r["K"])) == shape]
        add(max(rows, key=lambda r: float(r["tflops"])), "BASELINE config, fastest row")
    return out


CONFIG_COLUMNS = ["predicted_label", "model_label", "tag", "M", "N", "K"] + KEY_FIELDS + \
    ["regsPerThread", "theoretical_waves_per_cu", "pred_tflops", "measured_tflops"]
CONFIG_COLUMNS_2 = CONFIG_COLUMNS + ["schedule", "why"]


def cmd_select(args):
    reg = REGISTRATIONS[args.registration]
    if reg.number == "design":
        rows = design_configs()
        note = "label-design set (in-sample, never scored); see ridge_amd/labelcheck.py design_configs"
    elif reg.number in TABLE_RULE_REGISTRATIONS:
        rows = select_configs3(reg)
        note = "registered before any rocprofv3 run; see %s" % os.path.relpath(reg.mapping, ROOT)
    else:
        rows = select_configs(reg.sources, reg.hw_json, registration=reg.number)
        note = "registered before any rocprofv3 run; see %s" % os.path.relpath(reg.mapping, ROOT)
    cols = CONFIG_COLUMNS if reg.number == 1 else CONFIG_COLUMNS_2
    out = args.out or reg.configs
    T.write(out, cols, rows, [note])
    for r in rows:
        print("%-9s %-28s %6dx%-6dx%-5d %dx%dx%d w%dx%d s%d g%d %s" % (
            r["predicted_label"], r["tag"], r["M"], r["N"], r["K"], *[r[k] for k in KEY_FIELDS], r.get("why", "")))
    print("wrote %d configs to %s" % (len(rows), out))


def load_configs(path=CONFIGS_CSV):
    rows = _read_rows(path)
    for r in rows:
        for k in ["M", "N", "K"] + KEY_FIELDS + ["regsPerThread", "theoretical_waves_per_cu"]:
            r[k] = int(r[k])
    return rows


def cmd_run(args):
    """The launches rocprofv3 observes: per config and per K multiplier of its
    registration (`Registration.factors`, the multiplier 1 first), LAUNCHES
    launches of the registered variant at that K, each followed by a
    synchronize."""
    import torch
    from ridge_amd import gemm as G
    reg = REGISTRATIONS[args.registration]
    configs = load_configs(args.configs or reg.configs)
    dev = "cuda:0"
    for i, c in enumerate(configs):
        idx = G.find_variant(*[c[k] for k in KEY_FIELDS])
        if idx < 0:
            raise SystemExit("config %d: variant not in the kernel table (a row retired after the "
                             "registration; its counters were gathered and scored before, and a replay "
                             "needs the table of the registration commit)" % i)
        for factor in reg.factors(c):
            M, N, K = c["M"], c["N"], int(c["K"] * factor)
            if not G.variant(idx).divides(M, N, K):
                raise SystemExit("config %d: variant does not divide %dx%dx%d" % (i, M, N, K))
            print("config %d/%d %s %dx%dx%d %s" % (i + 1, len(configs), c["predicted_label"], M, N, K,
                                                   G.variant(idx).label()), flush=True)
            torch.cuda.synchronize()
            A = torch.empty((M, K), dtype=torch.float16, device=dev)
            B = torch.empty((K, N), dtype=torch.float16, device=dev)
            C = torch.empty((M, N), dtype=torch.float16, device=dev)
            G.fill_uniform(A, 1)
            G.fill_uniform(B, 2)
            torch.cuda.synchronize()
            for _ in range(args.launches):
                rc = G.launch(idx, A, B, C, M, N, K)
                if rc != 0:
                    raise SystemExit("config %d: launch returned %d" % (i, rc))
                torch.cuda.synchronize()
            del A, B, C
    print("labelcheck run: %d configs x %d launches at each of their K multipliers" % (len(configs), args.launches),
          flush=True)


# ---------------------------------------------------------------------------
# Parsing rocprofv3 CSV output.
# ---------------------------------------------------------------------------

# Kernel names as rocprofv3 reports them: Itanium-mangled, each int template
# argument as Li<n>E (gemmMfmaKernelILi64ELi64E...), or demangled (<64, 64, ...>).
_GEMM_NAME = re.compile(r"gemmMfma(?:PingPong|Persistent)?Kernel(?:I" + r"Li(\d+)E" * 7 + r"|<" +
                        r",".join([r"\s*(\d+)"] * 7) + r"\s*>)")


def _template_args(name):
    m = _GEMM_NAME.search(name)
    vals = [g for g in m.groups() if g is not None]
    return tuple(int(x) for x in vals)


def gemm_dispatches(parsed, configs, launches):
    """The GEMM dispatches in dispatch order, grouped per config: `launches`
    dispatches per config (an int for all, or one count per config, as when
    configs are launched at different numbers of K multipliers); each name must
    carry that config's template arguments."""
    counts = [launches] * len(configs) if isinstance(launches, int) else list(launches)
    gemm = [(k, v) for k, v in sorted(parsed.items()) if _GEMM_NAME.search(v["name"])]
    if len(gemm) != sum(counts):
        raise SystemExit("expected %d GEMM dispatches, found %d" % (sum(counts), len(gemm)))
    groups = []
    at = 0
    for i, c in enumerate(configs):
        chunk = gemm[at:at + counts[i]]
        at += counts[i]
        want = tuple(c[k] for k in KEY_FIELDS)
        for _, v in chunk:
            got = _template_args(v["name"])
            if got != want:
                raise SystemExit("config %d: dispatch of %s, expected %s" % (i, got, want))
        groups.append([v for _, v in chunk])
    return groups


def cmd_gather(args):
    reg = REGISTRATIONS[args.registration]
    configs = load_configs(args.configs or reg.configs)
    # The design set has no frozen calibration: the XCD count is the chip's.
    hw_json = reg.hw_json if os.path.exists(reg.hw_json) else os.path.join(ROOT, "data", "hardware", "mi355x.json")
    with open(hw_json) as f:
        hwj = json.load(f)
    xcds = int(hwj.get("numXcds", 8))
    facs = [reg.factors(c) for c in configs]
    per = [args.launches * len(f) for f in facs]
    p1 = gemm_dispatches(parse_counter_dir(args.counters), configs, per)
    pf = gemm_dispatches(parse_counter_dir(args.fetch), configs, per)
    pw = gemm_dispatches(parse_counter_dir(args.write), configs, per)
    pt = gemm_dispatches(parse_trace_dir(args.trace), configs, per)
    n = args.launches
    rows = []
    cols = CONFIG_COLUMNS if reg.number == 1 else CONFIG_COLUMNS_2
    dcols = []
    for f in facs:
        dcols += [reg.duration_column(x) for x in f if reg.duration_column(x) not in dcols]
    for i, c in enumerate(configs):
        med = lambda xs: statistics.median(xs)  # noqa: E731
        row = {k: c[k] for k in cols}
        for name in PASS1_COUNTERS:
            # GRBM_* clock counts per XCD, every other counter summed over its
            # instances (rocprof.counter_value).
            row[name] = med([counter_value(d, name, xcds) for d in p1[i][:n]])
        row["FETCH_SIZE"] = med([counter_value(d, "FETCH_SIZE", xcds) for d in pf[i][:n]])
        row["WRITE_SIZE"] = med([counter_value(d, "WRITE_SIZE", xcds) for d in pw[i][:n]])
        for col in dcols:
            row[col] = ""
        for j, f in enumerate(facs[i]):
            row[reg.duration_column(f)] = med([d["ns"] for d in pt[i][j * n:(j + 1) * n]])
        rows.append(row)
    out = args.out or reg.counters
    T.write(out, list(rows[0].keys()), rows,
            ["rocprofv3 counters per registered config (medians over %d launches); GRBM counters per XCD" % n])
    print("wrote %d rows to %s" % (len(rows), out))


# ---------------------------------------------------------------------------
# Scoring: the registered table and nothing else.
# ---------------------------------------------------------------------------

def derived(row, hwj):
    """AMD's derived-counter definitions (rocprofiler-sdk counter_defs.yaml for
    gfx950: MfmaUtil, LdsUtil, OccupancyPercent, SIMD_UTILIZATION) plus HBM% from
    the scaled traffic counters over the kernel-trace duration."""
    cus = float(hwj["numSMs"])
    simds = cus * float(hwj.get("simdsPerSM", 4))
    gui = float(row["GRBM_GUI_ACTIVE"])
    count = float(row["GRBM_COUNT"])
    out = {}
    out["mfma_pct"] = 100.0 * float(row["SQ_VALU_MFMA_BUSY_CYCLES"]) / (gui * simds)
    out["lds_pct"] = 100.0 * float(row["SQ_LDS_IDX_ACTIVE"]) / (gui * cus)
    out["occ_pct"] = 400.0 * float(row["SQ_WAVE_CYCLES"]) / gui / cus / float(hwj["maxWarpsPerSM"])
    out["simd_util_pct"] = 100.0 * float(row["SQ_BUSY_CU_CYCLES"]) / count / cus
    bytes_ = (float(row["FETCH_SIZE"]) * FETCH_SCALE + float(row["WRITE_SIZE"]) * WRITE_SCALE) * 1024.0
    out["hbm_tbs"] = bytes_ / (float(row["duration_ns"]) * 1e-9) / 1e12
    out["hbm_pct"] = 100.0 * out["hbm_tbs"] * 1e12 / float(hwj["hbmBytesPerSec"])
    out["theoretical_occ_pct"] = 100.0 * float(row["theoretical_waves_per_cu"]) / float(hwj["maxWarpsPerSM"])
    return out


def counter_label(d):
    """The registered decision table (rocprof-label-mapping.md section 2)."""
    if d["hbm_pct"] >= HBM_PCT_MIN:
        return "HBM"
    if d["simd_util_pct"] < SIMD_UTIL_PCT_MAX:
        return "WAVES"
    if d["occ_pct"] / d["theoretical_occ_pct"] < OCC_SHORTFALL_MAX:
        return "OCC"
    if d["lds_pct"] > d["mfma_pct"]:
        return "SMEM"
    if d["mfma_pct"] >= MFMA_PCT_MIN:
        return "TENSOR_CORE"
    return "ENVELOPE"


# Registration 2's decision table (data/sweep/rocprof-label2-mapping.md section 2).
STEADY_SHARE_MIN = 0.80     # rule 2: steady-state share below 0.80 -> ENVELOPE (or WAVES, the worse)


def derived2(row, hwj, long_factor):
    """Registration 2's quantities: registration 1's, with HBM% as the share of
    the launch the DRAM traffic needs at the calibrated read and write rates, and
    the steady-state share s = t(K x F) / (F t(K)), the launch's time at K against
    F times its time per K at K x F (where fill and drain are amortised)."""
    d = derived(row, hwj)
    read = float(row["FETCH_SIZE"]) * FETCH_SCALE * 1024.0
    write = float(row["WRITE_SIZE"]) * WRITE_SCALE * 1024.0
    dur = float(row["duration_ns"]) * 1e-9
    d["hbm_pct"] = 100.0 * (read / float(hwj["hbmBytesPerSec"]) + write / float(hwj["hbmWriteBytesPerSec"])) / dur
    d["steady_share"] = float(row["long_duration_ns"]) / (long_factor * float(row["duration_ns"]))
    return d


def counter_label2(d):
    """Registration 2's table, first match wins; a row no rule claims is
    UNDECIDED (scored as a disagreement: there is no fall-through label)."""
    if d["hbm_pct"] >= HBM_PCT_MIN:
        return "HBM"
    busy = d["simd_util_pct"] / 100.0
    if d["steady_share"] < STEADY_SHARE_MIN or busy < SIMD_UTIL_PCT_MAX / 100.0:
        return "ENVELOPE" if d["steady_share"] < busy else "WAVES"
    if d["occ_pct"] / d["theoretical_occ_pct"] < OCC_SHORTFALL_MAX:
        return "OCC"
    if d["lds_pct"] > d["mfma_pct"]:
        return "SMEM"
    if d["mfma_pct"] >= MFMA_PCT_MIN:
        return "TENSOR_CORE"
    return "UNDECIDED"


# Registration 3's decision table (data/sweep/rocprof-label3-mapping.md section 3),
# first match wins. The model's labelModel 1 applies the same table to its own
# prediction of these quantities.
DRAM_SHARE_MIN_3 = 0.70      # rule 1: DRAM share >= 0.70                        -> HBM
CU_SHARE_MIN_3 = 0.55        # rule 2: CU share < 0.55                           -> WAVES
BODY_SHARE_MIN_3 = 0.60      # rule 3: body share < 0.60                         -> ENVELOPE
LDS_OVER_MFMA_MIN_3 = 0.70   # rule 4: LDS share >= 0.70 x MFMA share            -> SMEM
MFMA_OVER_BODY_MIN_3 = 0.60  # rule 5: MFMA share / min(1, body share) >= 0.60   -> TENSOR_CORE
                             # rule 6: otherwise                                 -> OCC
CONTROL_CU_SHARE_3 = (0.70, 1.05)


def derived3(row, hwj):
    """Registration 3's quantities, each over the kernel-trace duration of the
    launch at K, none over the counters' own collection window (which runs several
    microseconds past a short kernel): the SQ cycle counts are converted at the
    launch's clock, its GRBM cycles over its duration, capped at the engine's
    nominal clock. The body share comes from the duration at the second K of
    body_factors."""
    cus = float(hwj["numSMs"])
    simds = cus * float(hwj.get("simdsPerSM", 4))
    dur = float(row["duration_ns"]) * 1e-9
    clock = min(float(row["GRBM_GUI_ACTIVE"]) / dur, float(hwj["nominalClockHz"]))
    read = float(row["FETCH_SIZE"]) * FETCH_SCALE * 1024.0
    write = float(row["WRITE_SIZE"]) * WRITE_SCALE * 1024.0
    d = {"clock_hz": clock, "duration_us": dur * 1e6}
    d["dram_share"] = (read / float(hwj["hbmBytesPerSec"]) + write / float(hwj["hbmWriteBytesPerSec"])) / dur
    d["mfma_share"] = float(row["SQ_VALU_MFMA_BUSY_CYCLES"]) / (simds * dur * clock)
    d["lds_share"] = float(row["SQ_LDS_IDX_ACTIVE"]) / (cus * dur * clock)
    d["cu_share"] = float(row["SQ_BUSY_CU_CYCLES"]) / (cus * dur * clock)
    f = body_factors({"K": int(row["K"]), "BK": int(row["BK"])})[1]
    t2 = float(row[Registration.duration_column(REGISTRATIONS[3], f)]) * 1e-9
    d["body_factor"] = f
    d["body_share"] = (t2 - dur) / ((f - 1.0) * dur)
    return d


def counter_label3(d):
    """Registration 3's table, first match wins. Also applied, in a test, to the
    model's predicted quantities, which must give the model's own label."""
    if d["dram_share"] >= DRAM_SHARE_MIN_3:
        return "HBM"
    if d["cu_share"] < CU_SHARE_MIN_3:
        return "WAVES"
    if d["body_share"] < BODY_SHARE_MIN_3:
        return "ENVELOPE"
    if d["lds_share"] >= LDS_OVER_MFMA_MIN_3 * d["mfma_share"]:
        return "SMEM"
    if d["mfma_share"] / min(1.0, d["body_share"]) >= MFMA_OVER_BODY_MIN_3:
        return "TENSOR_CORE"
    return "OCC"


def score(rows, hwj, registration=1):
    """(results, agree, need, control_ok): results over every row, the count of
    scored rows (the control excluded) whose counter label equals the model's,
    the registered pass threshold, and whether the control's SIMD utilisation
    is in its band (if not, the normalisations are wrong and the run is void)."""
    results = []
    control_ok = True
    reg = REGISTRATIONS[registration]
    for r in rows:
        if registration in TABLE_RULE_REGISTRATIONS:
            d = derived3(r, hwj)
            results.append((r, d, counter_label3(d)))
            if r["predicted_label"] == "CONTROL":
                lo, hi = CONTROL_CU_SHARE_3
                control_ok = control_ok and lo <= d["cu_share"] <= hi
            continue
        if registration == 2:
            d = derived2(r, hwj, reg.long_factor)
            results.append((r, d, counter_label2(d)))
        else:
            d = derived(r, hwj)
            results.append((r, d, counter_label(d)))
        if r["predicted_label"] == "CONTROL":
            lo, hi = CONTROL_SIMD_UTIL_PCT
            control_ok = control_ok and lo <= d["simd_util_pct"] <= hi
    scored = [x for x in results if x[0]["predicted_label"] != "CONTROL"]
    agree = sum(1 for r, d, lab in scored if lab == r["predicted_label"])
    need = -(-int(PASS_FRACTION * 100) * len(scored) // 100)
    return results, agree, need, control_ok


def relabel_in_sample(rows, hw_path):
    """Counters already seen, relabelled: each row's label from the model with the
    calibration at hw_path, against registration 3's table on the same row's
    counters (converted with that calibration's rates). The table and the model
    terms were developed on such rows, so the agreement is an in-sample figure and
    never the result of a check. Returns score()'s tuple, with no pass threshold."""
    with open(hw_path) as f:
        hwj = json.load(f)
    hw = RM.Hardware(hw_path)
    results = []
    for r in rows:
        label = "CONTROL" if r["predicted_label"] == "CONTROL" else predict_row(hw, r, True)["bottleneck"]
        d = derived3(r, hwj)
        results.append((dict(r, predicted_label=label), d, counter_label3(d)))
    agree = sum(1 for r, d, lab in results if r["predicted_label"] != "CONTROL" and lab == r["predicted_label"])
    return results, agree, None, True


def _print_score3(results, agree, need, control_ok):
    print("%-11s %-20s %-26s %8s %5s %5s %5s %5s %5s %5s  %-11s" % (
        "model", "shape", "variant", "us", "DRAM", "CU", "body", "LDS", "MFMA", "GHz", "counters"))
    by_label = {}
    for r, d, lab in results:
        shape = "%sx%sx%s" % (r["M"], r["N"], r["K"])
        var = "%sx%sx%s w%sx%s s%s g%s" % tuple(r[k] for k in KEY_FIELDS)
        verdict = "" if r["predicted_label"] == "CONTROL" else (
            "agree" if lab == r["predicted_label"] else "DISAGREE")
        print("%-11s %-20s %-26s %8.1f %5.2f %5.2f %5.2f %5.2f %5.2f %5.2f  %-11s %s" % (
            r["predicted_label"], shape, var, d["duration_us"], d["dram_share"], d["cu_share"], d["body_share"],
            d["lds_share"], d["mfma_share"], d["clock_hz"] / 1e9, lab, verdict))
        if r["predicted_label"] != "CONTROL":
            s = by_label.setdefault(r["predicted_label"], [0, 0])
            s[0] += lab == r["predicted_label"]
            s[1] += 1
    print()
    for lab in LABEL_ORDER_3:
        if lab in by_label:
            print("  %-11s %d of %d agree" % (lab, by_label[lab][0], by_label[lab][1]))
    if not control_ok:
        print("\ncontrol CU share outside [%g, %g]: the normalisations are wrong, the run is VOID" % CONTROL_CU_SHARE_3)
        return 2
    scored = sum(1 for r, d, lab in results if r["predicted_label"] != "CONTROL")
    if need is None:
        print("\n%d of %d configs agree (in-sample relabelling, not a check result)" % (agree, scored))
        return 0
    verdict = "PASS" if agree >= need else "FAIL"
    print("\n%d of %d configs agree (registered pass: >= %d) -> %s" % (agree, scored, need, verdict))
    return 0 if verdict == "PASS" else 1


def cmd_score(args):
    reg = REGISTRATIONS[args.registration]
    if args.relabel_hw or reg.number == "design":
        hw_path = args.relabel_hw or os.path.join(ROOT, "data", "hardware", "mi355x.json")
        rows = _read_rows(args.counters_csv or reg.counters)
        return _print_score3(*relabel_in_sample(rows, hw_path))
    with open(reg.hw_json) as f:
        hwj = json.load(f)
    rows = _read_rows(args.counters_csv or reg.counters)
    results, agree, need, control_ok = score(rows, hwj, reg.number)
    if reg.number in TABLE_RULE_REGISTRATIONS:
        return _print_score3(results, agree, need, control_ok)
    print("%-9s %-28s %-22s %6s %6s %6s %6s %6s %6s %6s  %-9s" % (
        "model", "shape", "variant", "HBM%", "SIMD%", "occ%", "theo%", "LDS%", "MFMA%", "steady", "counters"))
    by_label = {}
    for r, d, lab in results:
        shape = "%sx%sx%s" % (r["M"], r["N"], r["K"])
        var = "%sx%sx%s w%sx%s s%s g%s" % tuple(r[k] for k in KEY_FIELDS)
        verdict = "" if r["predicted_label"] == "CONTROL" else (
            "agree" if lab == r["predicted_label"] else "DISAGREE")
        print("%-9s %-28s %-22s %6.1f %6.1f %6.1f %6.1f %6.1f %6.1f %6s  %-9s %s" % (
            r["predicted_label"], shape, var, d["hbm_pct"], d["simd_util_pct"], d["occ_pct"],
            d["theoretical_occ_pct"], d["lds_pct"], d["mfma_pct"],
            "%.3f" % d["steady_share"] if "steady_share" in d else "-", lab, verdict))
        if r["predicted_label"] == "CONTROL":
            continue
        s = by_label.setdefault(r["predicted_label"], [0, 0])
        s[0] += lab == r["predicted_label"]
        s[1] += 1
    print()
    for lab in LABEL_ORDER:
        if lab in by_label:
            print("  %-9s %d of %d agree%s" % (lab, by_label[lab][0], by_label[lab][1],
                                              "  (fall-through label: weakest evidence)"
                                              if lab == "ENVELOPE" and reg.number == 1 else ""))
    if not control_ok:
        print("\ncontrol SIMD utilisation outside [%g, %g]%%: the normalisations are wrong, the run is VOID"
              % CONTROL_SIMD_UTIL_PCT)
        return 2
    scored = sum(1 for r, d, lab in results if r["predicted_label"] != "CONTROL")
    verdict = "PASS" if agree >= need else "FAIL"
    print("\n%d of %d configs agree (registered pass: >= %d) -> %s" % (agree, scored, need, verdict))
    return 0 if verdict == "PASS" else 1


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--registration", type=lambda x: x if x == "design" else int(x), default=CURRENT,
                    choices=list(REGISTRATIONS))
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("select")
    s.add_argument("--out", default=None)
    r = sub.add_parser("run")
    r.add_argument("--configs", default=None)
    r.add_argument("--launches", type=int, default=LAUNCHES)
    g = sub.add_parser("gather")
    g.add_argument("--configs", default=None)
    g.add_argument("--launches", type=int, default=LAUNCHES)
    for k in ("counters", "fetch", "write", "trace"):
        g.add_argument("--" + k, required=True)
    g.add_argument("--out", default=None)
    c = sub.add_parser("score")
    c.add_argument("--counters-csv", default=None)
    c.add_argument("--relabel-hw", default=None,
                   help="relabel the counters with the current model and this calibration "
                        "(in-sample; the design set always is)")
    args = ap.parse_args(argv)
    return {"select": cmd_select, "run": cmd_run, "gather": cmd_gather, "score": cmd_score}[args.cmd](args)


if __name__ == "__main__":
    sys.exit(main() or 0)
