"""The rocprofv3 label check's registration, selection, parsing and decision
table, on the CPU (the counters themselves come from the GPU box)."""
import csv
import os
import re

import pytest

from ridge_amd import labelcheck as LC

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REG = os.path.join(ROOT, "data", "sweep", "rocprof-label-mapping.md")


def test_committed_config_list_is_the_registered_selection(tmp_path):
    """Re-running the registered selection gives the committed configs and labels
    (measured_tflops is informational: the value the sweep held at registration)."""
    out = tmp_path / "c.csv"
    LC.main(["--registration", "1", "select", "--out", str(out)])
    keep = [c for c in LC.CONFIG_COLUMNS if c != "measured_tflops"]
    now = [{k: r[k] for k in keep} for r in LC._read_rows(str(out))]
    committed = [{k: r[k] for k in keep} for r in LC._read_rows(LC.CONFIGS_CSV)]
    assert now == committed


def test_selection_rule_distinct_shapes_per_label():
    rows = LC.load_configs()
    assert rows[0]["predicted_label"] == "CONTROL"
    scored = rows[1:]
    labels = [r["predicted_label"] for r in scored]
    for lab in set(labels):
        shapes = [(r["M"], r["N"], r["K"]) for r in scored if r["predicted_label"] == lab]
        assert len(shapes) == len(set(shapes)) <= LC.PER_LABEL
        assert all(r["model_label"] == lab for r in scored if r["predicted_label"] == lab)
    # Groups appear in the registered order, each sorted by tag then tile.
    order = [LC.LABEL_ORDER.index(x) for x in labels]
    assert order == sorted(order)


def _d(**kw):
    base = dict(hbm_pct=10.0, simd_util_pct=99.0, occ_pct=25.0, theoretical_occ_pct=25.0, lds_pct=20.0,
                mfma_pct=50.0)
    base.update(kw)
    return base


def test_decision_table_first_match_wins():
    assert LC.counter_label(_d()) == "ENVELOPE"
    assert LC.counter_label(_d(hbm_pct=70.0, simd_util_pct=10.0)) == "HBM"
    assert LC.counter_label(_d(hbm_pct=69.9, simd_util_pct=79.9)) == "WAVES"
    assert LC.counter_label(_d(occ_pct=17.4, theoretical_occ_pct=25.0)) == "OCC"     # 0.696
    assert LC.counter_label(_d(occ_pct=17.6, theoretical_occ_pct=25.0)) == "ENVELOPE"  # 0.704
    assert LC.counter_label(_d(lds_pct=50.1, mfma_pct=50.0)) == "SMEM"
    assert LC.counter_label(_d(lds_pct=50.0, mfma_pct=50.0)) == "ENVELOPE"            # not strictly greater
    assert LC.counter_label(_d(mfma_pct=70.0)) == "TENSOR_CORE"
    # WAVES is decided before SMEM: an idle machine with a busy LDS is WAVES.
    assert LC.counter_label(_d(simd_util_pct=50.0, lds_pct=90.0)) == "WAVES"


def test_registration_text_matches_the_code():
    text = open(REG).read()
    assert re.search(r"\| 1 \| HBM% ≥ (\d+) \| `HBM` \|", text).group(1) == "%g" % LC.HBM_PCT_MIN
    assert re.search(r"\| 2 \| SIMD% < (\d+) \| `WAVES` \|", text).group(1) == "%g" % LC.SIMD_UTIL_PCT_MAX
    assert float(re.search(r"\| 3 \| occ% / theoretical occ% < ([0-9.]+) \| `OCC` \|", text).group(1)) == \
        LC.OCC_SHORTFALL_MAX
    assert "| 4 | LDS% > MFMA% | `SMEM` |" in text
    assert re.search(r"\| 5 \| MFMA% ≥ (\d+) \| `TENSOR_CORE` \|", text).group(1) == "%g" % LC.MFMA_PCT_MIN
    assert "At least %d%% of the" % int(LC.PASS_FRACTION * 100) in text
    n = len(LC.load_configs()) - 1
    assert "%d scored configs (%d of %d)" % (n, -(-75 * n // 100), n) in text


def test_derived_quantities_use_amd_definitions():
    hwj = {"numSMs": 256, "simdsPerSM": 4, "maxWarpsPerSM": 32, "hbmBytesPerSec": 5e12}
    row = {"GRBM_GUI_ACTIVE": 1000.0, "GRBM_COUNT": 1000.0, "SQ_VALU_MFMA_BUSY_CYCLES": 512000.0,
           "SQ_LDS_IDX_ACTIVE": 64000.0, "SQ_WAVE_CYCLES": 512000.0, "SQ_BUSY_CU_CYCLES": 256000.0,
           "FETCH_SIZE": 1000.0, "WRITE_SIZE": 500.0, "duration_ns": 1000.0, "theoretical_waves_per_cu": 8}
    d = LC.derived(row, hwj)
    assert d["mfma_pct"] == pytest.approx(50.0)      # 512000 / (1000 * 1024)
    assert d["lds_pct"] == pytest.approx(25.0)       # 64000 / (1000 * 256)
    # 8 waves per CU for 1000 cycles = 2000 wave-quad-cycles per CU, x 256 CUs:
    # 400 * 512000 / 1000 / 256 / 32 = 25% of the 32 wave slots
    assert d["occ_pct"] == pytest.approx(25.0)
    assert d["simd_util_pct"] == pytest.approx(100.0)
    assert d["theoretical_occ_pct"] == pytest.approx(25.0)
    # (1000 * 2 + 500) KiB in 1 us = 2.56 GB/ms = 2.56 TB/s
    assert d["hbm_tbs"] == pytest.approx(2500 * 1024 / 1e-6 / 1e12)


def _write_counter_csv(path, dispatches):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for did, name, counters in dispatches:
            for cn, vals in counters.items():
                for v in vals:
                    w.writerow([did, name, cn, v])


def test_gather_groups_dispatches_by_order_and_checks_names(tmp_path):
    configs = [dict(M=256, N=256, K=64, BM=64, BN=64, BK=32, WM=32, WN=32, stages=4, groupM=8),
               dict(M=512, N=512, K=64, BM=128, BN=128, BK=32, WM=64, WN=64, stages=4, groupM=8)]
    # one demangled and one mangled name, as rocprofv3 may report either
    names = ["void ridge::gemmMfmaKernel<64, 64, 32, 32, 32, 4, 8>(_Float16 const*)",
             "_ZN5ridge14gemmMfmaKernelILi128ELi128ELi32ELi64ELi64ELi4ELi8EEEvPKDF16_S2_PDF16_iii"]
    disp = [(1, "fillUniformKernel", {"GRBM_GUI_ACTIVE": [5.0]})]
    did = 2
    for c, n in zip(configs, names):
        for j in range(2):
            disp.append((did, n, {"GRBM_GUI_ACTIVE": [100.0 * did] * 8}))
            did += 1
    d = tmp_path / "p" / "host" / "123"
    d.mkdir(parents=True)
    _write_counter_csv(d / "run_counter_collection.csv", disp)
    groups = LC.gemm_dispatches(LC.parse_counter_dir(str(tmp_path / "p")), configs, 2)
    assert [len(g) for g in groups] == [2, 2]
    # eight per-XCD rows: the max is the per-XCD count
    assert LC.counter_value(groups[1][0], "GRBM_GUI_ACTIVE", 8) == 400.0
    bad = [dict(configs[0]), dict(configs[1], groupM=4)]
    with pytest.raises(SystemExit, match="expected"):
        LC.gemm_dispatches(LC.parse_counter_dir(str(tmp_path / "p")), bad, 2)
    with pytest.raises(SystemExit, match="expected 6 GEMM dispatches"):
        LC.gemm_dispatches(LC.parse_counter_dir(str(tmp_path / "p")), configs, 3)


def test_committed_counters_score_as_reported():
    """The committed counters through the registered table give the reported
    result (5 of 13, FAIL; control in band) and the per-label split."""
    import json
    with open(LC.HW_JSON) as f:
        hwj = json.load(f)
    rows = LC._read_rows(LC.COUNTERS_CSV)
    results, agree, need, control_ok = LC.score(rows, hwj)
    assert control_ok and (agree, need) == (5, 10)
    split = {}
    for r, d, lab in results:
        if r["predicted_label"] != "CONTROL":
            s = split.setdefault(r["predicted_label"], [0, 0])
            s[0] += lab == r["predicted_label"]
            s[1] += 1
    assert split == {"SMEM": [0, 4], "WAVES": [4, 4], "ENVELOPE": [0, 4], "HBM": [1, 1]}


REG2 = LC.REGISTRATIONS[2]


def test_registration_2_committed_configs_are_its_selection(tmp_path):
    """Registration 2's committed config list re-derives from its frozen files,
    holds every required config, and is the control plus 21 scored configs."""
    out = tmp_path / "c2.csv"
    LC.main(["--registration", "2", "select", "--out", str(out)])
    keep = [c for c in LC.CONFIG_COLUMNS_2 if c != "measured_tflops"]
    now = [{k: r[k] for k in keep} for r in LC._read_rows(str(out))]
    committed = [{k: r[k] for k in keep} for r in LC._read_rows(REG2.configs)]
    assert now == committed
    rows = LC.load_configs(REG2.configs)
    assert rows[0]["predicted_label"] == "CONTROL" and len(rows) == 22
    keys = {tuple(r[k] for k in ["M", "N", "K"] + LC.KEY_FIELDS) for r in rows[1:]}
    for key, _why in LC.REQUIRED_2:
        assert key in keys
    assert all(r["model_label"] == r["predicted_label"] for r in rows[1:])


def _d2(**kw):
    base = dict(hbm_pct=10.0, simd_util_pct=99.0, occ_pct=25.0, theoretical_occ_pct=25.0, lds_pct=20.0,
                mfma_pct=50.0, steady_share=0.95)
    base.update(kw)
    return base


def test_registration_2_decision_table():
    assert LC.counter_label2(_d2()) == "UNDECIDED"                          # no fall-through label
    assert LC.counter_label2(_d2(hbm_pct=70.0, steady_share=0.1)) == "HBM"
    assert LC.counter_label2(_d2(steady_share=0.79)) == "ENVELOPE"
    assert LC.counter_label2(_d2(steady_share=0.80)) == "UNDECIDED"
    assert LC.counter_label2(_d2(simd_util_pct=79.0)) == "WAVES"            # s 0.95 > 0.79
    assert LC.counter_label2(_d2(simd_util_pct=60.0, steady_share=0.5)) == "ENVELOPE"   # the worse of the two
    assert LC.counter_label2(_d2(simd_util_pct=40.0, steady_share=0.5)) == "WAVES"
    assert LC.counter_label2(_d2(occ_pct=17.4)) == "OCC"
    assert LC.counter_label2(_d2(lds_pct=50.1, mfma_pct=50.0)) == "SMEM"
    assert LC.counter_label2(_d2(mfma_pct=70.0)) == "TENSOR_CORE"


def test_registration_2_derived_quantities():
    """HBM% at the two calibrated rates and the steady-state share."""
    hwj = {"numSMs": 256, "simdsPerSM": 4, "maxWarpsPerSM": 32, "hbmBytesPerSec": 8e12,
           "hbmWriteBytesPerSec": 4e12}
    row = {"GRBM_GUI_ACTIVE": 1000.0, "GRBM_COUNT": 1000.0, "SQ_VALU_MFMA_BUSY_CYCLES": 512000.0,
           "SQ_LDS_IDX_ACTIVE": 64000.0, "SQ_WAVE_CYCLES": 512000.0, "SQ_BUSY_CU_CYCLES": 256000.0,
           "FETCH_SIZE": 1000.0, "WRITE_SIZE": 500.0, "duration_ns": 1000.0, "long_duration_ns": 12800.0,
           "theoretical_waves_per_cu": 8}
    d = LC.derived2(row, hwj, 16)
    # reads 2000 KiB at 8 TB/s + writes 500 KiB at 4 TB/s, over 1 us
    assert d["hbm_pct"] == pytest.approx(100.0 * (2048000 / 8e12 + 512000 / 4e12) / 1e-6)
    assert d["steady_share"] == pytest.approx(12800.0 / (16 * 1000.0))


def test_registration_2_text_matches_the_code():
    text = open(REG2.mapping).read()
    assert "| 1 | HBM%% ≥ %g | `HBM` |" % LC.HBM_PCT_MIN in text
    assert "| 2 | s < %.2f or SIMD%% < %g |" % (LC.STEADY_SHARE_MIN, LC.SIMD_UTIL_PCT_MAX) in text
    assert "| 6 | otherwise | `UNDECIDED` (a disagreement) |" in text
    n = len(LC.load_configs(REG2.configs)) - 1
    assert "%d scored configs (%d of %d)" % (n, -(-75 * n // 100), n) in text
    assert "K × %d" % REG2.long_factor in text


def test_registration_2_counters_score_as_reported():
    """Registration 2's committed counters through its registered table: 8 of 21
    agree, FAIL (16 needed); the control is in band."""
    import json
    with open(REG2.hw_json) as f:
        hwj = json.load(f)
    rows = LC._read_rows(REG2.counters)
    results, agree, need, control_ok = LC.score(rows, hwj, 2)
    assert control_ok and (agree, need) == (8, 16)
    split = {}
    for r, d, lab in results:
        if r["predicted_label"] != "CONTROL":
            s = split.setdefault(r["predicted_label"], [0, 0])
            s[0] += lab == r["predicted_label"]
            s[1] += 1
    assert split == {"SMEM": [0, 4], "WAVES": [3, 4], "ENVELOPE": [2, 5], "HBM": [3, 8]}


REG3 = LC.REGISTRATIONS[3]


def test_registration_3_configs_are_its_selection(tmp_path):
    """Registration 3's committed config list re-derives from its frozen files
    (the fifth held-out sweep's shapes, the frozen table and calibration): the
    control, the three BASELINE rows, then at most four configs of distinct
    shapes per label in the registered order, every one labelled so by the model."""
    out = tmp_path / "c3.csv"
    LC.main(["--registration", "3", "select", "--out", str(out)])
    now = LC._read_rows(str(out))
    committed = LC._read_rows(REG3.configs)
    assert now == committed
    rows = LC.load_configs(REG3.configs)
    assert rows[0]["predicted_label"] == "CONTROL"
    assert [r["why"] for r in rows[1:4]] == ["required: BASELINE config, best row"] * 3
    fresh = rows[4:]
    labels = [r["predicted_label"] for r in fresh]
    assert [LC.LABEL_ORDER_3.index(x) for x in labels] == sorted(LC.LABEL_ORDER_3.index(x) for x in labels)
    for lab in set(labels):
        shapes = [(r["M"], r["N"], r["K"]) for r in fresh if r["predicted_label"] == lab]
        assert len(shapes) == len(set(shapes)) <= LC.PER_LABEL
    assert all(r["model_label"] == r["predicted_label"] for r in rows[1:])
    heldout = {(m, n, k) for m, n, k, _ in LC.T.read_shapes(LC.HELDOUT5_SHAPES)}
    assert all((r["M"], r["N"], r["K"]) in heldout for r in fresh)
    assert len(rows) - 1 == 26


def test_registration_3_body_factor_rule():
    assert LC.body_factors({"K": 4096, "BK": 32}) == [1, 0.5]
    assert LC.body_factors({"K": 128, "BK": 64}) == [1, 0.5]     # one K tile at K / 2
    assert LC.body_factors({"K": 128, "BK": 128}) == [1, 2]      # K / 2 is half a tile
    assert LC.body_factors({"K": 192, "BK": 64}) == [1, 2]       # 96 is not a whole tile


def _d3(**kw):
    base = dict(dram_share=0.3, cu_share=0.9, body_share=0.9, lds_share=0.2, mfma_share=0.7)
    base.update(kw)
    return base


def test_registration_3_decision_table():
    assert LC.counter_label3(_d3()) == "TENSOR_CORE"
    assert LC.counter_label3(_d3(dram_share=0.70, cu_share=0.1, body_share=0.1)) == "HBM"
    assert LC.counter_label3(_d3(cu_share=0.549, body_share=0.1)) == "WAVES"   # WAVES before ENVELOPE
    assert LC.counter_label3(_d3(cu_share=0.55, body_share=0.599)) == "ENVELOPE"
    assert LC.counter_label3(_d3(lds_share=0.49)) == "SMEM"                     # 0.49 >= 0.7 x 0.7
    assert LC.counter_label3(_d3(lds_share=0.48)) == "TENSOR_CORE"
    # MFMA share over the body share (capped at 1): 0.48 / 0.8 = 0.6.
    assert LC.counter_label3(_d3(mfma_share=0.48, body_share=0.8, lds_share=0.1)) == "TENSOR_CORE"
    assert LC.counter_label3(_d3(mfma_share=0.47, body_share=0.8, lds_share=0.1)) == "OCC"
    assert LC.counter_label3(_d3(mfma_share=0.59, body_share=1.3, lds_share=0.1)) == "OCC"


def test_registration_3_derived_quantities():
    """Shares over the kernel-trace duration at the launch's clock (GRBM cycles
    over the duration, capped at the nominal clock), and the two-point body share."""
    hwj = {"numSMs": 256, "simdsPerSM": 4, "hbmBytesPerSec": 8e12, "hbmWriteBytesPerSec": 4e12,
           "nominalClockHz": 2.4e9}
    row = {"K": 4096, "BK": 32, "duration_ns": 100000.0, "duration_x0.5_ns": 55000.0,
           "GRBM_GUI_ACTIVE": 180000.0, "SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 90000.0,
           "SQ_LDS_IDX_ACTIVE": 256 * 36000.0, "SQ_BUSY_CU_CYCLES": 256 * 162000.0,
           "FETCH_SIZE": 100000.0, "WRITE_SIZE": 50000.0}
    d = LC.derived3(row, hwj)
    assert d["clock_hz"] == pytest.approx(1.8e9)                       # 180,000 cycles in 100 us
    assert d["mfma_share"] == pytest.approx(0.5)
    assert d["lds_share"] == pytest.approx(0.2)
    assert d["cu_share"] == pytest.approx(0.9)
    assert d["body_share"] == pytest.approx((55000 - 100000) / (-0.5 * 100000))   # 0.9
    assert d["dram_share"] == pytest.approx((100000 * 2048 / 8e12 + 50000 * 1024 / 4e12) / 1e-4)
    short = dict(row, GRBM_GUI_ACTIVE=480000.0)                          # 4.8 GHz: the window, not the kernel
    assert LC.derived3(short, hwj)["clock_hz"] == 2.4e9


def test_registration_3_text_matches_the_code():
    text = open(REG3.mapping).read()
    assert "| 1 | DRAM share ≥ %.2f | `HBM` |" % LC.DRAM_SHARE_MIN_3 in text
    assert "| 2 | CU share < %.2f | `WAVES` |" % LC.CU_SHARE_MIN_3 in text
    assert "| 3 | body share < %.2f | `ENVELOPE` |" % LC.BODY_SHARE_MIN_3 in text
    assert "| 4 | LDS share ≥ %.2f x MFMA share | `SMEM` |" % LC.LDS_OVER_MFMA_MIN_3 in text
    assert "| 5 | MFMA share / min(1, body share) ≥ %.2f | `TENSOR_CORE` |" % LC.MFMA_OVER_BODY_MIN_3 in text
    assert "| 6 | otherwise | `OCC` |" in text
    n = len(LC.load_configs(REG3.configs)) - 1
    assert "%d scored configs (%d of %d)" % (n, -(-75 * n // 100), n) in text
    assert "[%.2f, %.2f]" % LC.CONTROL_CU_SHARE_3 in text
    import json
    assert json.load(open(REG3.hw_json)) == json.load(open(os.path.join(ROOT, "data", "sweep",
                                                                         "mi355x-heldout5-hw.json")))


def test_registration_3_counters_score_as_reported():
    """Registration 3's committed counters through its registered table: 19 of 26
    agree, FAIL (20 needed); 17 of the 23 held-out configs; the control in band."""
    import json
    with open(REG3.hw_json) as f:
        hwj = json.load(f)
    rows = LC._read_rows(REG3.counters)
    results, agree, need, control_ok = LC.score(rows, hwj, 3)
    assert control_ok and (agree, need) == (19, 20)
    split = {}
    for r, d, lab in results:
        if r["predicted_label"] != "CONTROL":
            s = split.setdefault(r["predicted_label"], [0, 0])
            s[0] += lab == r["predicted_label"]
            s[1] += 1
    assert split == {"HBM": [4, 5], "WAVES": [4, 4], "ENVELOPE": [3, 4], "SMEM": [4, 5], "TENSOR_CORE": [0, 4],
                     "OCC": [4, 4]}
    fresh = [(r, lab) for r, d, lab in results if r["why"] == "per-label rule"]
    assert len(fresh) == 23 and sum(lab == r["predicted_label"] for r, lab in fresh) == 17


REG4 = LC.REGISTRATIONS[4]


def test_registration_4_configs_are_its_selection(tmp_path):
    """Registration 4 re-derives from its frozen files with registration 3's rule
    (the sixth held-out sweep, the same frozen table); its text is registration
    3's table, quantities and criterion."""
    out = tmp_path / "c4.csv"
    LC.main(["--registration", "4", "select", "--out", str(out)])
    assert LC._read_rows(str(out)) == LC._read_rows(REG4.configs)
    rows = LC.load_configs(REG4.configs)
    assert rows[0]["predicted_label"] == "CONTROL" and len(rows) - 1 == 26
    heldout = {(m, n, k) for m, n, k, _ in LC.T.read_shapes(REG4.heldout_shapes)}
    assert all((r["M"], r["N"], r["K"]) in heldout for r in rows[4:])
    assert all(r["model_label"] == r["predicted_label"] for r in rows[1:])
    assert LC._read_rows(REG4.table) == LC._read_rows(REG3.table)
    text3, text4 = open(REG3.mapping).read(), open(REG4.mapping).read()
    for start, end in (("## 3. Decision procedure", "**Control.**"), ("## 5. Pass criterion", "## 6.")):
        sec = lambda t: t[t.index(start):t.index(end)]  # noqa: E731
        assert sec(text4).replace("labelModel 2", "labelModel 1") == sec(text3)
    import json
    hw4 = json.load(open(REG4.hw_json))
    assert hw4["labelModel"] == 2 and hw4 == json.load(open(os.path.join(ROOT, "data", "sweep",
                                                                         "mi355x-heldout6-hw.json")))
    hw3 = json.load(open(REG3.hw_json))
    assert {k: v for k, v in hw4.items() if k != "labelModel"} == {k: v for k, v in hw3.items() if k != "labelModel"}


def test_registration_4_counters_score_as_reported():
    """Registration 4's committed counters through the registered table: 22 of 26
    agree, PASS (20 needed); 20 of the 23 held-out configs; the control in band."""
    import json
    with open(REG4.hw_json) as f:
        hwj = json.load(f)
    rows = LC._read_rows(REG4.counters)
    results, agree, need, control_ok = LC.score(rows, hwj, 4)
    assert control_ok and (agree, need) == (22, 20)
    split = {}
    for r, d, lab in results:
        if r["predicted_label"] != "CONTROL":
            s = split.setdefault(r["predicted_label"], [0, 0])
            s[0] += lab == r["predicted_label"]
            s[1] += 1
    assert split == {"HBM": [4, 4], "WAVES": [4, 4], "ENVELOPE": [2, 5], "SMEM": [4, 5], "TENSOR_CORE": [4, 4],
                     "OCC": [4, 4]}
    fresh = [(r, lab) for r, d, lab in results if r["why"] == "per-label rule"]
    assert len(fresh) == 23 and sum(lab == r["predicted_label"] for r, lab in fresh) == 20


def test_in_sample_relabelling_figures():
    """The in-sample figures the registrations quote, from committed counters: the
    design set (61 configs, never scored) agrees on 55 under the current model and
    under registration 3's frozen calibration; registration 3's counters, relabelled
    by the current model, agree on 22 of 26 (their registered score stays 19; 21
    before mallWriteModel)."""
    design = LC._read_rows(LC.REGISTRATIONS["design"].counters)
    assert len(design) == 61 and all(r["predicted_label"] == "DESIGN" for r in design)
    current = os.path.join(ROOT, "data", "hardware", "mi355x.json")
    for hw in (current, REG3.hw_json):
        results, agree, need, _ = LC.relabel_in_sample(design, hw)
        assert (agree, need) == (55, None)
    results, agree, _, _ = LC.relabel_in_sample(LC._read_rows(REG3.counters), current)
    assert agree == 22 and sum(r["predicted_label"] != "CONTROL" for r, d, lab in results) == 26
