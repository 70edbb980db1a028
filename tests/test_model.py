"""The cost model (no GPU).

A100 mode: the reference's hand-derived worked example and invariants
(test/test-model.cpp:47-181), and byte-identical batch output against the
reference's own model build on the reference's 336-row sweep.
CDNA4 mode: a hand-derived worked example in the same style; the test follows
the derivation, never the code.
"""
import filecmp
import math
import os
import subprocess

import pytest

from ridge_amd import model as RM

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="module")
def a100():
    return RM.Hardware("a100")


@pytest.fixture(scope="module")
def mi355x():
    return RM.Hardware("mi355x")


@pytest.fixture(scope="module")
def mi355x_calibrated():
    return RM.Hardware(os.path.join(ROOT, "data", "hardware", "mi355x.json"))


def test_a100_worked_example(a100):
    # test-model.cpp:47-101, values derived by hand there.
    p = RM.predict(a100, M=4096, N=4096, K=4096, BM=128, BN=128, BK=32, warpM=64, warpN=64, stages=3,
                   regsPerThread=128)
    assert p["numWarps"] == 4
    assert p["tComputeCycles"] == pytest.approx(512.0, abs=1e-6)
    assert p["tSmemCycles"] == pytest.approx(256.0, abs=1e-6)
    assert p["tStepCycles"] == pytest.approx(768.0, abs=1e-6)
    assert p["smEfficiency"] == pytest.approx(512.0 / 768.0, abs=1e-9)
    assert p["ctasPerSM"] == 3
    assert p["occFactor"] == pytest.approx(0.75, abs=1e-9)
    assert p["totalCtas"] == pytest.approx(1024.0)
    assert p["ctaSlots"] == pytest.approx(324.0)
    assert p["wavesExact"] == pytest.approx(1024.0 / 324.0, abs=1e-9)
    assert p["waveEfficiency"] == pytest.approx(1024.0 / 1296.0, abs=1e-9)
    assert p["kSteps"] == pytest.approx(128.0)
    assert p["tPrologueCycles"] == pytest.approx(831.651840, abs=1e-4)
    assert p["tEpilogueCycles"] == pytest.approx(1663.303680, abs=1e-4)
    assert p["tBodyCycles"] == pytest.approx(98304.0, abs=1e-6)
    assert p["envelopeEfficiency"] == pytest.approx(0.975248, abs=1e-6)
    assert p["peakTensorTFLOPS"] == pytest.approx(311.869440, abs=1e-3)
    assert p["computeTFLOPS"] == pytest.approx(120.158068, abs=1e-4)
    assert p["baseIntensity"] == pytest.approx(64.0)
    assert p["l2ReuseFactor"] == pytest.approx(18.0)
    assert p["arithmeticIntensity"] == pytest.approx(1152.0)
    assert p["hbmTFLOPS"] == pytest.approx(2304.0, abs=1e-6)
    assert p["predictedTFLOPS"] == pytest.approx(120.158068, abs=1e-4)
    assert p["bottleneck"] == "SMEM"


def test_a100_sub_wave_grid(a100):
    # test-model.cpp:103-124: 16 CTAs in 324 slots.
    p = RM.predict(a100, M=512, N=512, K=4096, BM=128, BN=128, BK=32, warpM=64, warpN=64, stages=3,
                   regsPerThread=128)
    assert p["totalCtas"] == 16 and p["ctaSlots"] == 324
    assert p["waveEfficiency"] == pytest.approx(16 / 324, abs=1e-9)
    assert p["predictedTFLOPS"] == pytest.approx(7.509879, abs=1e-4)
    assert p["bottleneck"] == "WAVES"


def test_a100_invariants(a100):
    # test-model.cpp:126-181.
    assert 250 < RM.predict(a100)["peakTensorTFLOPS"] < 400
    p = RM.predict(a100, M=8192, N=8192, K=8192)
    assert 0 < p["predictedTFLOPS"] <= p["computeTFLOPS"] + 1e-6 and p["predictedTFLOPS"] <= p["hbmTFLOPS"] + 1e-6
    assert 0 < p["occFactor"] <= 1 and 0 < p["envelopeEfficiency"] <= 1 and p["ctasPerSM"] >= 1
    assert 0 < p["smEfficiency"] < 1
    big = RM.predict(a100, BM=256, BN=256, warpM=64, warpN=64)
    small = RM.predict(a100, BM=64, BN=64, warpM=64, warpN=64)
    assert big["baseIntensity"] > small["baseIntensity"]
    deep = dict(M=4096, N=4096, K=4096, BM=128, BN=128, BK=32, warpM=64, warpN=64, stages=3, regsPerThread=128)
    pd = RM.predict(a100, **deep)
    ps = RM.predict(a100, **dict(deep, K=128))
    assert ps["envelopeEfficiency"] < pd["envelopeEfficiency"] and ps["kSteps"] < pd["kSteps"]
    assert ps["bottleneck"] == "ENVELOPE"
    assert RM.predict(a100, BM=512, BN=512, BK=128, stages=8)["bottleneck"] == "DOES_NOT_FIT"


@pytest.mark.parametrize("hw,fixture", [
    ("tests/golden/a100-sxm4-40gb.json", "a100_predictions_ref_calibrated.csv"),
    ("a100", "a100_predictions_ref_placeholder.csv"),
])
def test_a100_batch_byte_identical_to_reference_model(tmp_path, hw, fixture):
    """Same pred_* strings (6 significant digits) and hence the same ranking and
    tie structure as the reference's own model on its 336-row sweep."""
    out = tmp_path / "pred.csv"
    RM.predict_batch(os.path.join(GOLD, "a100_measured.csv"), str(out),
                     hw=os.path.join(ROOT, hw) if hw.endswith(".json") else hw)
    assert filecmp.cmp(str(out), os.path.join(GOLD, fixture), shallow=False)
    ref_bin = os.path.join(ROOT, "oracle", "_ref", "ridge-predict")
    if os.path.exists(ref_bin):  # the live reference build, where it exists
        live = tmp_path / "live.csv"
        cmd = [ref_bin] + (["--hw", os.path.join(ROOT, hw)] if hw.endswith(".json") else ["--gpu", hw])
        subprocess.run(cmd + ["--batch", os.path.join(GOLD, "a100_measured.csv"), "--out", str(live)],
                       check=True, capture_output=True)
        assert filecmp.cmp(str(out), str(live), shallow=False)


def test_mi355x_worked_example(mi355x):
    """4096^3, 256x256x64 tile, 128x64 wavefront tile, 2 stages, 214 registers, on
    the MI355X placeholders. Derivation:

      waves          (256/128) x (256/64) = 8, 512 workitems
      MFMA/wave/step (128/16) x (64/16) x (64/32) = 64
      tCompute       64 x 8 waves x 4 cycles = 2048
      tSmem          8 x (128 + 64) x 64 x 2 B = 196608 B / 128 = 1536
      tStep          3584, smEff 2048/3584 = 0.571429
      LDS            2 x (256x64 + 64x256) x 2 = 131072 -> floor(163840/131072) = 1
      wave slots     floor(32/8) = 4
      registers      214 -> 216 (granule 8); floor(512/216) = 2 waves/SIMD;
                     8 waves over 4 SIMDs = 2 per SIMD -> 1 workgroup
      workgroups/CU  1, occ min(1, 8/8) = 1
      grid           16 x 16 = 256 in 256 slots: waveEff 1
      gmem B/cycle   8e12 / (2.4e9 x 256) = 13.0208333
      prologue       1 x 65536 / 13.0208333 = 5033.1648
      epilogue       256 x 256 x 2 / 13.0208333 = 10066.3296
      body           64 K-steps x 3584 = 229376
      envelope       229376 / 244475.4944 = 0.938237
      peak           16384 / 4 x 2.4e9 x 256 = 2516.5824 TFLOP/s
      compute        2516.5824 x 0.571429 x 0.938237 = 1349.22
      base AI        2 x 256 x 256 x 4096 / ((256 + 256) x 4096 x 2) = 128
      launch order   256 tiles, all resident, 32 per XCD: XCD 0 runs logical ids
                     0..31; groupM 8 (the config default): group = 8 rows x 16
                     columns, ids 0..31 -> rows 0..7 (id % 8), columns 0..3 (id / 8)
                     -> 8 A panels + 4 B panels; AI = 2 x 32 x 256^2 x 4096 /
                     ((8 + 4) x 256 x 4096 x 2) = 682.667
      compulsory     2 x 4096^3 / (3 x 4096^2 x 2) = 1365.33; AI = 682.667
      HBM            8e12 x 682.667 = 5461.33 TFLOP/s; label SMEM (0.571 worst)
    """
    p = RM.predict(mi355x, M=4096, N=4096, K=4096, BM=256, BN=256, BK=64, warpM=128, warpN=64, stages=2,
                   regsPerThread=214)
    assert p["numWarps"] == 8
    assert p["tComputeCycles"] == pytest.approx(2048.0)
    assert p["tSmemCycles"] == pytest.approx(1536.0)
    assert p["smEfficiency"] == pytest.approx(2048 / 3584, abs=1e-9)
    assert p["ctasPerSM"] == 1 and p["occFactor"] == pytest.approx(1.0)
    assert p["ctaSlots"] == 256 and p["waveEfficiency"] == pytest.approx(1.0)
    assert p["tPrologueCycles"] == pytest.approx(5033.1648, abs=1e-3)
    assert p["tEpilogueCycles"] == pytest.approx(10066.3296, abs=1e-3)
    assert p["envelopeEfficiency"] == pytest.approx(0.938237, abs=1e-6)
    assert p["peakTensorTFLOPS"] == pytest.approx(2516.5824, abs=1e-6)
    assert p["computeTFLOPS"] == pytest.approx(2516.5824 * (2048 / 3584) * (229376 / 244475.4944), abs=1e-6)
    assert p["baseIntensity"] == pytest.approx(128.0)
    assert (p["reuseTilesM"], p["reuseTilesN"]) == (8.0, 4.0)
    assert p["arithmeticIntensity"] == pytest.approx(2048 / 3, abs=1e-9)
    assert p["compulsoryIntensity"] == pytest.approx(2 * 4096 / 6, abs=1e-9)
    assert p["hbmTFLOPS"] == pytest.approx(8 * 2048 / 3, abs=1e-6)
    assert p["bottleneck"] == "SMEM"


def test_compact_block_reuse_model(tmp_path):
    """l2ReuseModel 1 (the grid-bounded compact block, no launch order) on the
    worked example's config: 32 slots per XCD, a = floor(sqrt 32) = 5, b =
    ceil(32/5) = 7, a = ceil(32/7) = 5; AI = (5x256)(7x256)/((5+7)x256) = 746.667."""
    cfg = ('{"name": "x", "arch": "gfx950", "numSMs": 256, "clockHz": 2.4e9, "mmaCyclesPerInst": 4, '
           '"smemBytesPerCycle": 128, "hbmBytesPerSec": 8e12, "regsPerSM": 131072, "smemBytesPerSM": 163840, '
           '"maxWarpsPerSM": 32, "maxCtasPerSM": 32, "warpsNeededToHide": 8, "l2ReuseModel": 1}')
    f = tmp_path / "m1.json"
    f.write_text(cfg)
    p = RM.predict(RM.Hardware(str(f)), M=4096, N=4096, K=4096, BM=256, BN=256, BK=64, warpM=128, warpN=64,
                   stages=2, regsPerThread=214)
    assert (p["reuseTilesM"], p["reuseTilesN"]) == (5.0, 7.0)
    assert p["arithmeticIntensity"] == pytest.approx(1280 * 1792 / 3072, abs=1e-9)
    assert p["hbmTFLOPS"] == pytest.approx(8 * 1280 * 1792 / 3072, abs=1e-6)


def test_mi355x_ping_pong_overlap_and_prologue_of_existing_tiles(mi355x):
    """256x256x32 tile, 128x64 wavefront tile, 4 stages, 197 registers on the
    MI355X placeholders: 8 waves (two per SIMD) with >= 3 stages is the
    ping-pong schedule, whose operand reads run under the other wave's MFMAs.

      MFMA/wave/step (128/16) x (64/16) x (32/32) = 32
      tCompute       32 x 8 waves x 4 cycles = 1024
      tSmem          8 x (128 + 64) x 32 x 2 B = 98304 B / 128 = 768
      tStep          max(1024, 768) = 1024 -> smEff 1 (in series: 1792, 0.571429)

    At K = 64 only two K tiles exist: the prologue fills min(3, 2) = 2 of them,
    2 x (256x32 + 32x256) x 2 B / 13.0208333 B/cycle = 5033.1648 cycles (the
    reference's stages-1 rule would charge 3 tiles, 7549.7472)."""
    p = RM.predict(mi355x, M=4096, N=4096, K=4096, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=4,
                   regsPerThread=197)
    assert p["tComputeCycles"] == pytest.approx(1024.0)
    assert p["tSmemCycles"] == pytest.approx(768.0)
    assert p["tStepCycles"] == pytest.approx(1024.0)
    assert p["smEfficiency"] == pytest.approx(1.0)
    # Two stages: the uniform schedule, reads and MFMAs in series.
    p2 = RM.predict(mi355x, M=4096, N=4096, K=4096, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=2,
                    regsPerThread=197)
    assert p2["tStepCycles"] == pytest.approx(1792.0)
    # Four waves: no ping-pong even with 4 stages.
    p4 = RM.predict(mi355x, M=4096, N=4096, K=4096, BM=256, BN=128, BK=32, warpM=128, warpN=64, stages=4,
                    regsPerThread=197)
    # 32 MFMAs x 4 waves x 4 cycles + 4 x 192 x 32 x 2 B / 128 = 512 + 384.
    assert p4["tStepCycles"] == pytest.approx(896.0)
    short = RM.predict(mi355x, M=4096, N=4096, K=64, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=4,
                       regsPerThread=197)
    assert short["kSteps"] == 2
    assert short["tPrologueCycles"] == pytest.approx(5033.1648, abs=1e-3)
    ref = RM.predict(RM.Hardware("a100"), M=4096, N=4096, K=64, BM=256, BN=256, BK=32, warpM=64, warpN=64,
                     stages=4, regsPerThread=0)
    # A100 mode keeps the reference's rule: 3 tiles of (256x32 + 32x256) x 2 B at
    # the a100() placeholder's 2.0e12 / (1.41e9 x 108) B/cycle.
    gmem = 2.0e12 / (1.41e9 * 108)
    assert ref["tPrologueCycles"] == pytest.approx(3 * 32768 / gmem / ref["ctasPerSM"], rel=1e-12)


def test_mi355x_latency_hiding_uses_the_ilp8_column(tmp_path):
    """A wave with >= 8 independent accumulator chains per K-step needs the ILP-8
    column of the latency surface (4 waves here) instead of the default 8.
    256x128 tile of 128x64 wavefront tiles: 4 waves of (128/16)(64/16) = 32
    chains; 261 registers -> 264, floor(512/264) = 1 wave per SIMD -> 1 workgroup,
    4 resident waves: occ 4/4 = 1 (default need: 4/8 = 0.5). 64x64 tile of 32x32
    wavefront tiles: (32/16)(32/16) = 4 chains, so the default need of 8 holds."""
    cfg = ('{"name": "x", "arch": "gfx950", "numSMs": 256, "clockHz": 2.4e9, "mmaCyclesPerInst": 4, '
           '"smemBytesPerCycle": 128, "hbmBytesPerSec": 8e12, "regsPerSM": 131072, "smemBytesPerSM": 163840, '
           '"maxWarpsPerSM": 32, "maxCtasPerSM": 32, "warpsNeededToHide": 8%s}')
    with_ilp = tmp_path / "ilp.json"
    with_ilp.write_text(cfg % ', "warpsNeededToHideIlp8": 4')
    without = tmp_path / "no.json"
    without.write_text(cfg % "")
    big = dict(BM=256, BN=128, BK=32, warpM=128, warpN=64, stages=4, regsPerThread=261)
    assert RM.predict(RM.Hardware(str(with_ilp)), **big)["occFactor"] == pytest.approx(1.0)
    assert RM.predict(RM.Hardware(str(without)), **big)["occFactor"] == pytest.approx(0.5)
    # 64x64 w32x32, 4 stages of 64x32 + 32x64 halves = 32 KiB: 5 by LDS, 8 by
    # wave slots (32/4); 62 registers -> 64, 8 waves per SIMD -> 8 by registers;
    # 5 workgroups x 4 waves = 20 resident waves >= 8 either way.
    small = dict(BM=64, BN=64, BK=32, warpM=32, warpN=32, stages=4, regsPerThread=62)
    p = RM.predict(RM.Hardware(str(with_ilp)), **small)
    assert p["ctasPerSM"] == 5 and p["occFactor"] == pytest.approx(1.0)


def test_mi355x_launch_order_reuse_follows_groupm(mi355x):
    """8192 x 8192 x 1024, 256x256 tiles (32 x 32 = 1024 tiles), one workgroup per
    CU: 256 resident, 32 per XCD. XCD x runs logical ids x*128 .. x*128 + 31
    (xcdRemap: q = 1024 / 8 = 128). groupM = 1 (row-major): ids 0..31 are one row
    of tiles -> 1 A row panel + 32 B column panels per XCD; intensity
    2*32*256^2*1024 / ((1*256 + 32*256) * 1024 * 2) = 248.24 FLOP/B. groupM = 4:
    pidInGroup 0..31 -> rows 0..3, columns 0..7 -> 4 + 8 panels -> 682.67.
    groupM = 16: 16 rows x 2 columns -> 455.11. The HBM ceiling is the
    placeholder's 8e12 B/s times the intensity."""
    cfg = dict(M=8192, N=8192, K=1024, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=4, regsPerThread=197)
    want = {1: (1, 32, 2 * 32 * 256 * 256 / (33 * 256 * 2)), 4: (4, 8, 2 * 32 * 256 * 256 / (12 * 256 * 2)),
            16: (16, 2, 2 * 32 * 256 * 256 / (18 * 256 * 2))}
    for g, (rows, cols, ai) in want.items():
        p = RM.predict(mi355x, groupM=g, **cfg)
        assert (p["reuseTilesM"], p["reuseTilesN"]) == (rows, cols), g
        assert p["arithmeticIntensity"] == pytest.approx(ai, rel=1e-12), g
        assert p["hbmTFLOPS"] == pytest.approx(8e12 * ai / 1e12, rel=1e-12), g
    assert want[1][2] == pytest.approx(248.2424, abs=1e-4)
    # The A100 (reference) model ignores groupM.
    a100 = RM.Hardware("a100")
    assert RM.predict(a100, groupM=1, **cfg)["predictedTFLOPS"] == RM.predict(a100, groupM=8, **cfg)["predictedTFLOPS"]


def test_mi355x_register_occupancy_per_simd(mi355x):
    # 4 waves of 133+128 = 261 registers: 264 rounded, floor(512/264) = 1 wave per
    # SIMD; 4 waves over 4 SIMDs = 1 per SIMD -> 1 workgroup. At 74 registers:
    # floor(512/80) = 6 waves per SIMD -> 6 workgroups by registers, LDS (64 KiB
    # at 2 stages of 128x128x64) allows 2.
    p = RM.predict(mi355x, BM=256, BN=128, BK=64, warpM=128, warpN=64, stages=2, regsPerThread=261)
    assert p["ctasPerSM"] == 1
    p = RM.predict(mi355x, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2, regsPerThread=74)
    assert p["ctasPerSM"] == 2
    # 600 registers exceed the 512 budget: does not fit.
    assert RM.predict(mi355x, regsPerThread=600)["bottleneck"] == "DOES_NOT_FIT"


def test_mi355x_tall_skinny_reuse_bounded_by_grid(mi355x):
    # N = 128 with BN = 128: one column of tiles, so every tile reads its own A
    # panel; the per-XCD block is a x 1 and intensity cannot exceed the
    # compulsory 2MNK / bytes = 125.1 FLOP/B (the reference's sqrt(slots) would
    # claim ~1000+).
    p = RM.predict(mi355x, M=16384, N=128, K=8192, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2,
                   regsPerThread=74)
    assert p["reuseTilesN"] == 1
    comp = 2 * 16384 * 128 * 8192 / ((16384 * 8192 + 8192 * 128) * 2 + 16384 * 128 * 2)
    assert p["compulsoryIntensity"] == pytest.approx(comp)
    assert p["arithmeticIntensity"] <= comp + 1e-9
    sq = RM.predict(RM.Hardware("a100"), M=16384, N=128, K=8192, BM=128, BN=128, BK=64, warpM=64, warpN=64,
                    stages=2, regsPerThread=74)
    assert sq["arithmeticIntensity"] > 5 * p["arithmeticIntensity"]


def test_hardware_json_loader_is_all_or_nothing(tmp_path):
    good = tmp_path / "g.json"
    good.write_text('{"name": "x", "note": "mentions numSMs and clockHz in prose", "arch": "gfx950", '
                    '"numSMs": 256, "clockHz": 2.1e9, "mmaCyclesPerInst": 9.5, "smemBytesPerCycle": 200, '
                    '"hbmBytesPerSec": 6.5e12, "regsPerSM": 131072, "smemBytesPerSM": 163840, '
                    '"maxWarpsPerSM": 32, "maxCtasPerSM": 32, "warpsNeededToHide": 8}')
    hw = RM.Hardware(str(good))
    assert hw.calibrated and hw.name == "x"
    p = RM.predict(hw, BM=256, BN=256, BK=64, warpM=128, warpN=64, stages=2, regsPerThread=214)
    assert p["numWarps"] == 8 and p["reuseTilesM"] > 0   # gfx950 target description
    bad = tmp_path / "b.json"
    bad.write_text(good.read_text().replace('"smemBytesPerCycle": 200, ', ''))
    with pytest.raises(ValueError, match="smemBytesPerCycle"):
        RM.Hardware(str(bad))
    zero = tmp_path / "z.json"
    zero.write_text(good.read_text().replace('"clockHz": 2.1e9', '"clockHz": 0'))
    with pytest.raises(ValueError, match='"clockHz" must be positive'):
        RM.Hardware(str(zero))
    with pytest.raises(ValueError, match="cannot read"):
        RM.Hardware(str(tmp_path / "missing.json"))
    # The reader's own error model: every failure names the file and what is wrong.
    for text, why in [
        (good.read_text().replace('"numSMs": 256', '"numSMs": 256.5'), '"numSMs" must be an integer'),
        (good.read_text().replace('"numSMs": 256', '"numSMs": "many"'), '"numSMs" must be a number'),
        (good.read_text().replace('"clockHz": 2.1e9', '"clockHz": 2.1e9, "clockHz": 1e9'), "appears twice"),
        (good.read_text().replace('"name": "x"', '"name": {"a": 1}'), "nested objects"),
        (good.read_text().replace('"name": "x"', '"name": [1]'), "arrays"),
        (good.read_text() + " {}", "after the end"),
        (good.read_text().rstrip().rstrip("}"), "not closed"),
        (good.read_text().replace('"clockHz": 2.1e9', '"clockHz" 2.1e9'), "':' belongs after"),
        # A number in quotes, and forms strtod takes but JSON does not write.
        (good.read_text().replace('"numSMs": 256', '"numSMs": "256"'), '"numSMs" must be a number, found the string'),
        (good.read_text().replace('"clockHz": 2.1e9', '"clockHz": "2.1e9"'), '"clockHz" must be a number'),
        (good.read_text().replace('"numSMs": 256', '"numSMs": 0x100'), "neither a number"),
        (good.read_text().replace('"clockHz": 2.1e9', '"clockHz": 0x1p31'), "neither a number"),
        (good.read_text().replace('"clockHz": 2.1e9', '"clockHz": inf'), "neither a number"),
        (good.read_text().replace('"clockHz": 2.1e9', '"clockHz": 2.e9'), "neither a number"),
        # A term switch takes only the values the model defines.
        (good.read_text().replace('"numSMs": 256', '"numSMs": 256, "labelModel": 3'),
         "labelModel must be an integer from 0 to 2, found 3"),
        (good.read_text().replace('"numSMs": 256', '"numSMs": 256, "launchModel": 2'),
         "launchModel must be an integer from 0 to 1, found 2"),
        (good.read_text().replace('"numSMs": 256', '"numSMs": 256, "l2ReuseModel": -1'),
         "l2ReuseModel must be an integer from 0 to 2, found -1"),
    ]:
        broken = tmp_path / "broken.json"
        broken.write_text(text)
        with pytest.raises(ValueError, match=why):
            RM.Hardware(str(broken))


def test_mi355x_persistent_rows_walk_tiles_and_pay_one_fill_and_drain(mi355x):
    """8192 x 8192 x 128, 128x128x64 tile, 64x64 wavefront tile, 4 stages, 185
    registers, schedule 2 (persistent store-behind) on the MI355X placeholders.

      compute waves  (128/64) x (128/64) = 4, plus 2 loader waves = 6
      MFMA/wave/step (64/16) x (64/16) x (64/32) = 32 -> tCompute 32 x 4 x 4 = 512
      tSmem          4 x (64 + 64) x 64 x 2 B = 65536 B / 128 = 512
      tStep          512 + 512 = 1024 (no ping-pong), smEff 0.5
      LDS            ring 4 x (128x64 + 64x128) x 2 = 131072, staging 4 waves x 16
                     rows x 4 tile-rows x 64 x 2 B = 32768 -> 163840 -> 1 per CU
      registers      185 -> 192; floor(512/192) = 2 waves/SIMD; 6 waves over 4
                     SIMDs = 2 per SIMD -> 1 workgroup
      latency        4 compute waves x 1 / 8 needed = 0.5 (placeholders measure no
                     ILP-8 column)
      grid           64 x 64 = 4096 tiles over 256 slots = 16 tiles per slot
      prologue       min(3, 128/64) = 2 tiles x 32768 B / 13.0208333 = 5033.1648
      epilogue       128 x 128 x 2 / 13.0208333 = 2516.5824
      envelope       16 x 2048 / (5033.1648 + 16 x 2048 + 2516.5824) = 0.812744
                     (schedule -1, one tile per workgroup: 2048 / 9597.7472 = 0.213383)
      compute        2516.5824 x 0.5 x 0.5 x 1 x 0.812744 = 511.334
      HBM            compulsory 2 x 8192^2 x 128 / ((2 x 8192 x 128 + 8192^2) x 2)
                     = 124.1212 FLOP/B -> 8e12 x 124.1212 = 992.97 TFLOP/s
    """
    cfg = dict(M=8192, N=8192, K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=4, regsPerThread=185,
               groupM=8)
    p = RM.predict(mi355x, schedule=2, **cfg)
    assert p["numWarps"] == 4 and p["ctasPerSM"] == 1
    assert p["tStepCycles"] == pytest.approx(1024.0) and p["smEfficiency"] == pytest.approx(0.5)
    assert p["occFactor"] == pytest.approx(0.5)
    assert p["wavesExact"] == pytest.approx(16.0) and p["waveEfficiency"] == pytest.approx(1.0)
    assert p["tPrologueCycles"] == pytest.approx(5033.1648, abs=1e-3)
    assert p["tEpilogueCycles"] == pytest.approx(2516.5824, abs=1e-3)
    assert p["envelopeEfficiency"] == pytest.approx(32768 / 40317.7472, abs=1e-9)
    assert p["computeTFLOPS"] == pytest.approx(2516.5824 * 0.25 * 32768 / 40317.7472, abs=1e-6)
    assert p["compulsoryIntensity"] == pytest.approx(17179869184 / 138412032, abs=1e-9)
    assert p["hbmTFLOPS"] == pytest.approx(8 * 17179869184 / 138412032, abs=1e-6)
    assert p["predictedTFLOPS"] == pytest.approx(p["computeTFLOPS"])
    one = RM.predict(mi355x, schedule=-1, **cfg)
    assert one["envelopeEfficiency"] == pytest.approx(2048 / 9597.7472, abs=1e-9)
    # An explicit uniform schedule is the derived one for a 4-wave row.
    assert RM.predict(mi355x, schedule=0, **cfg) == one


def test_mi355x_persistent_occupancy_counts_loaders_and_staging(mi355x):
    """64x64x32 tile, 32x32 wavefront tiles (4 compute waves), registers unknown.
    Persistent: 6 waves -> floor(32/6) = 5 by wave slots; LDS ring + staging:
      s4: 4 x (64x32 + 32x64) x 2 = 32768 + 4 x 16 x 2 x 32 x 2 = 8192 -> 40960
          -> floor(163840/40960) = 4 (the ring alone would allow 5)
      s2: 16384 + 8192 = 24576 -> 6, so the wave slots bind: 5
    One tile per workgroup: 4 waves -> 8 slots; s4 LDS 32768 -> 5."""
    base = dict(M=4096, N=4096, K=4096, BM=64, BN=64, BK=32, warpM=32, warpN=32, regsPerThread=0)
    assert RM.predict(mi355x, stages=4, schedule=2, **base)["ctasPerSM"] == 4
    assert RM.predict(mi355x, stages=2, schedule=2, **base)["ctasPerSM"] == 5
    assert RM.predict(mi355x, stages=4, schedule=-1, **base)["ctasPerSM"] == 5
    # The A100 model has no persistent term: the schedule field is ignored.
    a100 = RM.Hardware("a100")
    assert RM.predict(a100, stages=4, schedule=2, **base) == RM.predict(a100, stages=4, schedule=-1, **base)


_CDNA4_JSON = ('{"name": "x", "arch": "gfx950", "numSMs": 256, "clockHz": 2.4e9, "mmaCyclesPerInst": 4, '
               '"smemBytesPerCycle": 128, "hbmBytesPerSec": 8e12, "regsPerSM": 131072, "smemBytesPerSM": 163840, '
               '"maxWarpsPerSM": 32, "maxCtasPerSM": 32, "warpsNeededToHide": 8%s}')


def test_lds_read_model_prices_each_operand_at_its_rate(tmp_path):
    """ldsReadModel 1 with A reads at 256 B/cycle and transposing B reads at 128:
    a 256x256x32 tile of eight wavefront tiles reads 8 x 32 x 2 B = 512 B per
    wavefront-tile row or column of fragments per K-step, so

      w128x64: 512 x (128/256 + 64/128) = 512       (blended 128 B/cycle: 768)
      w64x128: 512 x (64/256 + 128/128) = 640       (blended: 768, orientation-blind)

    and a model without the two rates is refused."""
    f = tmp_path / "lds.json"
    f.write_text(_CDNA4_JSON % ', "ldsReadModel": 1, "ldsAReadBytesPerCycle": 256, "ldsBTrReadBytesPerCycle": 128')
    hw = RM.Hardware(str(f))
    cfg = dict(M=4096, N=4096, K=4096, BM=256, BN=256, BK=32, stages=2, regsPerThread=197)
    assert RM.predict(hw, warpM=128, warpN=64, **cfg)["tSmemCycles"] == pytest.approx(512.0)
    assert RM.predict(hw, warpM=64, warpN=128, **cfg)["tSmemCycles"] == pytest.approx(640.0)
    blended = tmp_path / "blend.json"
    blended.write_text(_CDNA4_JSON % "")
    for wm, wn in ((128, 64), (64, 128)):
        assert RM.predict(RM.Hardware(str(blended)), warpM=wm, warpN=wn, **cfg)["tSmemCycles"] == pytest.approx(768.0)
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "ldsReadModel": 1, "ldsAReadBytesPerCycle": 256')
    with pytest.raises(ValueError, match="ldsReadModel 1"):
        RM.Hardware(str(bad))


def test_clock_model_runs_the_last_wave_at_its_busy_share_clock(tmp_path):
    """clockModel 1 with ratios 1.25 / 1.3 / 1.3 / 1.3 at 1/2 .. 1/16 of the CUs
    busy. 256x256x32 tiles, 128x64 wavefront tiles, 4 stages: 128 KiB of LDS, one
    workgroup per CU, 256 slots.

      256 tiles: one full wave, busy 1 -> ratio 1, compute unchanged
      128 tiles: busy 1/2 -> 1.25; waves 128 / ((0 + 1/1.25) x 256) = 0.625
                 against the quantisation's 0.5: compute x 1.25
      192 tiles: busy 3/4 -> x = log2(4/3) = 0.415037, ratio 1 + 0.25 x 0.415037
      320 tiles: two waves, the last with 64 busy (1/4) -> 1.3;
                 320 / ((1 + 1/1.3) x 256) = 0.706522 against 0.625
        8 tiles: busy 1/32, flat beyond 1/16 -> 1.3
    """
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % (', "clockModel": 1, "clockRatioHalfCus": 1.25, "clockRatioQuarterCus": 1.3, '
                                 '"clockRatioEighthCus": 1.3, "clockRatioSixteenthCus": 1.3'))
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % "")
    hw_on, hw_off = RM.Hardware(str(on)), RM.Hardware(str(off))
    tile = dict(K=4096, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=4, regsPerThread=197)
    cases = [((4096, 4096), 1.0, 1.0), ((2048, 4096), 1.25, 0.625),
             ((3072, 4096), 1 + 0.25 * math.log2(4 / 3), None), ((5120, 4096), 1.3, 320 / ((1 + 1 / 1.3) * 256)),
             ((512, 1024), 1.3, None)]
    for (m, n), ratio, clocked in cases:
        p_on = RM.predict(hw_on, M=m, N=n, **tile)
        p_off = RM.predict(hw_off, M=m, N=n, **tile)
        assert p_on["ctasPerSM"] == 1
        assert p_on["tailClockFactor"] == pytest.approx(ratio, rel=1e-12)
        assert p_off["tailClockFactor"] == 1.0
        # The quantisation figure (and so the label) is the reference's either way.
        assert p_on["waveEfficiency"] == p_off["waveEfficiency"]
        if clocked is not None:
            assert p_on["computeTFLOPS"] / p_off["computeTFLOPS"] == pytest.approx(
                clocked / p_off["waveEfficiency"], rel=1e-12)
    # one busy wave of a partly filled grid: compute scales by the ratio itself
    p_on = RM.predict(hw_on, M=2048, N=4096, **tile)
    p_off = RM.predict(hw_off, M=2048, N=4096, **tile)
    assert p_on["computeTFLOPS"] / p_off["computeTFLOPS"] == pytest.approx(1.25, rel=1e-12)
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "clockModel": 1, "clockRatioHalfCus": 1.25')
    with pytest.raises(ValueError, match="clockModel 1"):
        RM.Hardware(str(bad))


def test_l2_stream_model_adds_the_l2_served_tile_loads(tmp_path):
    """l2StreamModel 1 at 16384 B/cycle and 2.4 GHz (39.3216 TB/s), HBM 8 TB/s.
    16384 x 128 x 8192 with 128x64x64 tiles, groupM 8: 128 x 2 = 256 tiles, one per
    CU. Every tile loads (128 + 64) x 8192 x 2 B = 3 MiB: 768 MiB in all. Per XCD
    (32 tiles, 16 row panels x 2 column panels) the launch order fetches 16 A and
    2 B panels once, 8 x (16 x 128 + 2 x 64) x 8192 x 2 B = 285,212,672 B from HBM,
    which is also what l2ReuseModel 2 charges. The rest, 805,306,368 - 285,212,672
    = 520,093,696 B, are L2 hits:

      t = 285212672 / 8e12 + 520093696 / 39.3216e12 = 35.652 us + 13.227 us
      hbmTFLOPS = 2 x 16384 x 128 x 8192 / t = 703.0 (HBM alone: 963.8)"""
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % ', "l2StreamModel": 1, "l2HitBytesPerCycle": 16384, "l2ReuseModel": 2')
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % ', "l2ReuseModel": 2')
    cfg = dict(M=16384, N=128, K=8192, BM=128, BN=64, BK=64, warpM=64, warpN=32, stages=6, regsPerThread=131,
               groupM=8, schedule=2)
    p_on = RM.predict(RM.Hardware(str(on)), **cfg)
    p_off = RM.predict(RM.Hardware(str(off)), **cfg)
    flops = 2.0 * 16384 * 128 * 8192
    assert p_off["l2HitBytes"] == 0.0
    assert flops / p_off["arithmeticIntensity"] == pytest.approx(285212672.0, rel=1e-12)
    assert p_on["l2HitBytes"] == pytest.approx(520093696.0, rel=1e-12)
    t = 285212672.0 / 8e12 + 520093696.0 / (16384 * 2.4e9)
    assert p_on["hbmTFLOPS"] == pytest.approx(flops / t / 1e12, rel=1e-12)
    assert p_on["hbmTFLOPS"] == pytest.approx(703.0, abs=0.05)
    assert p_off["hbmTFLOPS"] == pytest.approx(963.8, abs=0.05)
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "l2StreamModel": 1')
    with pytest.raises(ValueError, match="l2StreamModel 1"):
        RM.Hardware(str(bad))


def test_power_model_derates_by_matrix_pipe_share(tmp_path):
    """powerModel 1 with loadedClockRatio 0.8: a row whose compute ceiling is a
    share u of the matrix-pipe peak runs at clock x (1 - 0.2 u). The headline
    tile at 4096^3 on the placeholders: smEff 1 (ping-pong), occupancy 1, one
    full wave, envelope e, so u = e and the ceiling becomes e x (1 - 0.2 e) x
    peak. A ratio above 1 (data movement that raises the clock) is refused."""
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % ', "powerModel": 1, "loadedClockRatio": 0.8')
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % "")
    cfg = dict(M=4096, N=4096, K=4096, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=4, regsPerThread=197)
    p_on = RM.predict(RM.Hardware(str(on)), **cfg)
    p_off = RM.predict(RM.Hardware(str(off)), **cfg)
    u = p_off["computeTFLOPS"] / p_off["peakTensorTFLOPS"]
    assert p_off["smEfficiency"] == 1.0 and p_off["waveEfficiency"] == 1.0
    assert u == pytest.approx(p_off["envelopeEfficiency"] * p_off["occFactor"], rel=1e-12)
    assert p_on["powerClockFactor"] == pytest.approx(1 - 0.2 * u, rel=1e-12)
    assert p_on["computeTFLOPS"] == pytest.approx(p_off["computeTFLOPS"] * (1 - 0.2 * u), rel=1e-12)
    assert p_off["powerClockFactor"] == 1.0
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "powerModel": 1, "loadedClockRatio": 1.2')
    with pytest.raises(ValueError, match="powerModel 1"):
        RM.Hardware(str(bad))


def test_uniform_overlap_model_hides_part_of_the_shorter_phase(tmp_path):
    """uniformOverlapModel 1 with freeRunningOverlap 0.75 on the placeholders
    (4 cycles per MFMA per CU, 128 B/cycle LDS): the 8-wave uniform 256x256x32
    w128x64 tile at 2 stages has tC = 1024, tS = 768 and runs
    1024 + 768 - 0.75 x 768 = 1216 cycles per K-step (in series: 1792). A 4-wave
    uniform workgroup (one wave per SIMD) and the ping-pong rows are unchanged;
    the 8-compute-wave persistent row is covered."""
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % ', "uniformOverlapModel": 1, "freeRunningOverlap": 0.75')
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % "")
    hw_on, hw_off = RM.Hardware(str(on)), RM.Hardware(str(off))
    eight = dict(M=4096, N=4096, K=4096, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=2, regsPerThread=197)
    assert RM.predict(hw_off, **eight)["tStepCycles"] == pytest.approx(1792.0)
    assert RM.predict(hw_on, **eight)["tStepCycles"] == pytest.approx(1216.0)
    four = dict(eight, BN=128)
    assert RM.predict(hw_on, **four)["tStepCycles"] == RM.predict(hw_off, **four)["tStepCycles"]
    pp = dict(eight, stages=4)
    assert RM.predict(hw_on, **pp)["tStepCycles"] == pytest.approx(1024.0)
    # The 8-compute-wave persistent row (256x128x32 w64x64, schedule 2): its
    # compute waves run the same uniform loop, two per SIMD: tC = 16 MFMAs x 8
    # waves x 4 = 512, tS = 8 x (64 + 64) x 32 x 2 B / 128 = 512, so
    # 512 + 512 - 0.75 x 512 = 640 cycles (in series: 1024).
    pers = dict(M=8192, N=8192, K=128, BM=256, BN=128, BK=32, warpM=64, warpN=64, stages=6, regsPerThread=167,
                groupM=4, schedule=2)
    assert RM.predict(hw_off, **pers)["tStepCycles"] == pytest.approx(1024.0)
    assert RM.predict(hw_on, **pers)["tStepCycles"] == pytest.approx(640.0)
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "uniformOverlapModel": 1, "freeRunningOverlap": 1.5')
    with pytest.raises(ValueError, match="uniformOverlapModel 1"):
        RM.Hardware(str(bad))


def test_mall_stream_model_stretches_the_k_step_with_launch_order_misses(tmp_path):
    """mallStreamModel 1 on the placeholders (4 cycles per MFMA, 128 B/cycle LDS,
    2.4 GHz), MALL path 8 TB/s, stretch curve (load: stretch) 0: 1, 0.5: 1,
    1.0: 1.1, 1.5: 1.5, 2.0: 2.0. 8192 x 8192 x 4096, 256x256x32 w128x64 s4
    ping-pong, one workgroup per CU: tC = 32 MFMAs x 8 waves x 4 = 1024 cycles,
    tS = 8 x 192 x 64 / 128 = 768, K-step max = 1024 cycles = 426.67 ns.
    256 tiles resident, 32 per XCD (XCD x holds logical ids 128x .. 128x+31):
      groupM 1: one tile row, 32 columns: 1 + 32 panels per XCD, 8 + 256 in all;
        misses per K-step (8 x 256 + 256 x 256) x 32 x 2 B = 4,325,376 B,
        load 4,325,376 / 8e12 / 426.67 ns = 1.26720, stretch 1.1 + 0.4 x
        0.2672 / 0.5 = 1.31376, miss share 67,584 / (256 x 512) = 0.515625;
      groupM 4: 4 rows x 8 columns: 32 + 64 panels in all: 1,572,864 B,
        load 0.46080, stretch 1, miss share 0.1875."""
    curve = (', "mallStreamModel": 1, "mallRefillBytesPerSec": 8e12, '
             '"mallStretchLoad0": 0, "mallStretchLoad1": 0.5, "mallStretchLoad2": 1.0, "mallStretchLoad3": 1.5, '
             '"mallStretchLoad4": 2.0, "mallStretch0": 1, "mallStretch1": 1, "mallStretch2": 1.1, '
             '"mallStretch3": 1.5, "mallStretch4": 2.0')
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % curve)
    hw = RM.Hardware(str(on))
    cfg = dict(M=8192, N=8192, K=4096, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=4, regsPerThread=197,
               schedule=1)
    g1 = RM.predict(hw, groupM=1, **cfg)
    assert g1["refillMissShare"] == pytest.approx(0.515625)
    assert g1["mallLoad"] == pytest.approx(4325376 / 8e12 / (1024 / 2.4e9))
    assert g1["mallStretch"] == pytest.approx(1.1 + 0.4 * (g1["mallLoad"] - 1.0) / 0.5)
    assert g1["mallStretch"] == pytest.approx(1.31376, abs=1e-5)
    assert g1["tStepCycles"] == pytest.approx(1024 * g1["mallStretch"])
    g4 = RM.predict(hw, groupM=4, **cfg)
    assert g4["refillMissShare"] == pytest.approx(0.1875)
    assert g4["mallLoad"] == pytest.approx(0.4608, abs=1e-6) and g4["mallStretch"] == 1.0
    assert g4["tStepCycles"] == pytest.approx(1024.0)
    assert g1["predictedTFLOPS"] < g4["predictedTFLOPS"]
    # Beyond the last point the path's bandwidth binds: stretch proportional to load.
    steep = tmp_path / "steep.json"
    steep.write_text(_CDNA4_JSON % curve.replace('"mallRefillBytesPerSec": 8e12', '"mallRefillBytesPerSec": 4e12'))
    g1s = RM.predict(RM.Hardware(str(steep)), groupM=1, **cfg)
    assert g1s["mallLoad"] == pytest.approx(2 * g1["mallLoad"])
    assert g1s["mallStretch"] == pytest.approx(2.0 * g1s["mallLoad"] / 2.0)
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % curve.replace('"mallStretchLoad2": 1.0', '"mallStretchLoad2": 0.4'))
    with pytest.raises(ValueError, match="mallStreamModel 1"):
        RM.Hardware(str(bad))


def test_hbm_write_model_prices_c_at_the_write_rate(tmp_path):
    """hbmWriteModel 1 with reads at 8 TB/s and writes at 4 TB/s, on one XCD so
    that the 256 resident 128x128 tiles of 2048 x 2048 x 128 fetch every panel
    once: reads (2048 x 128 x 2) x 2 = 1,048,576 B, C 2048^2 x 2 = 8,388,608 B,
    2^30 FLOP: 1,048,576 / 8e12 + 8,388,608 / 4e12 = 2.228224 us, 481.882
    TFLOP/s (one rate for all 9,437,184 B: 910.222)."""
    base = ', "numXcds": 1'
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % base)
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % (base + ', "hbmWriteModel": 1, "hbmWriteBytesPerSec": 4e12'))
    cfg = dict(M=2048, N=2048, K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2, regsPerThread=128)
    flops = 2.0 * 2048 * 2048 * 128
    p_off = RM.predict(RM.Hardware(str(off)), **cfg)
    p_on = RM.predict(RM.Hardware(str(on)), **cfg)
    assert p_off["hbmTFLOPS"] == pytest.approx(flops / (9437184 / 8e12) / 1e12)
    assert p_on["hbmTFLOPS"] == pytest.approx(flops / (1048576 / 8e12 + 8388608 / 4e12) / 1e12)
    assert p_on["hbmTFLOPS"] == pytest.approx(481.882, abs=1e-3)
    assert p_on["arithmeticIntensity"] == pytest.approx(flops / 9437184)
    # The drain of each tile moves at the write rate: twice the cycles.
    assert p_on["tEpilogueCycles"] == pytest.approx(2 * p_off["tEpilogueCycles"])


def test_write_overlap_model_overlaps_c_with_the_l2_served_loads(tmp_path):
    """writeOverlapModel 1 on the case above plus l2StreamModel 1: the 256 tiles
    load (128 + 128) x 128 x 2 B each, 16,777,216 B, of which 1,048,576 come from
    DRAM and 15,728,640 from the L2s. At 4096 B/cycle x 2.4 GHz the L2-served
    loads take 1.6 us; in series with the reads (0.131072 us) and the writes
    (2.097152 us) the launch takes 3.828224 us, 280.479 TFLOP/s. With the term the
    writes overlap them: 0.131072 + max(2.097152, 1.6) = 2.228224 us, 481.882. At
    2048 B/cycle the L2-served loads take 3.2 us and bind instead: 0.131072 + 3.2 =
    3.331072 us. The term needs both stream terms."""
    base = ', "numXcds": 1, "hbmWriteModel": 1, "hbmWriteBytesPerSec": 4e12, "l2StreamModel": 1'
    cfg = dict(M=2048, N=2048, K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2, regsPerThread=128)
    flops = 2.0 * 2048 * 2048 * 128
    pred = {}
    for name, extra in (("series", ', "l2HitBytesPerCycle": 4096'),
                        ("overlap", ', "l2HitBytesPerCycle": 4096, "writeOverlapModel": 1'),
                        ("l2bound", ', "l2HitBytesPerCycle": 2048, "writeOverlapModel": 1')):
        f = tmp_path / (name + ".json")
        f.write_text(_CDNA4_JSON % (base + extra))
        pred[name] = RM.predict(RM.Hardware(str(f)), **cfg)
    assert pred["series"]["l2HitBytes"] == pytest.approx(15728640.0)
    assert pred["series"]["hbmTFLOPS"] == pytest.approx(flops / 3.828224e-6 / 1e12)
    assert pred["overlap"]["hbmTFLOPS"] == pytest.approx(flops / 2.228224e-6 / 1e12)
    assert pred["overlap"]["hbmTFLOPS"] == pytest.approx(481.882, abs=1e-3)
    assert pred["l2bound"]["hbmTFLOPS"] == pytest.approx(flops / 3.331072e-6 / 1e12)
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "numXcds": 1, "writeOverlapModel": 1')
    with pytest.raises(ValueError, match="writeOverlapModel 1"):
        RM.Hardware(str(bad))


def test_mall_reuse_model_serves_refetches_from_the_mall(tmp_path):
    """mallReuseModel 1 with reads at 8 TB/s, writes at 4 TB/s and MALL hits at
    2 TB/s, 8 XCDs in the launch order (l2ReuseModel 2): the 256 resident 128x128
    tiles of 2048 x 2048 x 128 (groupM 8) put 32 tiles on each XCD, 8 row panels
    by 4 column panels, so the XCDs fetch 8 x 12 x (128 x 128 x 2) = 3,145,728 B
    of A and B against 1,048,576 compulsory; C is 8,388,608 B. Without the term
    every fetch is a DRAM read: 3,145,728 / 8e12 + 8,388,608 / 4e12 = 2.490368 us.
    With it HBM reads each byte once and the other 2,097,152 B are MALL hits:
    1,048,576 / 8e12 + 2,097,152 / 2e12 + 8,388,608 / 4e12 = 3.2768 us."""
    base = ', "numXcds": 8, "l2ReuseModel": 2, "hbmWriteModel": 1, "hbmWriteBytesPerSec": 4e12'
    term = ', "mallReuseModel": 1, "mallRefillBytesPerSec": 2e12, "mallBytes": %d'
    cfg = dict(M=2048, N=2048, K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2, regsPerThread=128,
               groupM=8)
    flops = 2.0 * 2048 * 2048 * 128
    hw = {}
    for name, extra in (("off", ""), ("on", term % (256 << 20)), ("small", term % 1000000)):
        f = tmp_path / (name + ".json")
        f.write_text(_CDNA4_JSON % (base + extra))
        hw[name] = RM.Hardware(str(f))
    p_off, p_on, p_small = (RM.predict(hw[n], **cfg) for n in ("off", "on", "small"))
    assert (p_off["reuseTilesM"], p_off["reuseTilesN"]) == (8.0, 4.0)
    assert p_off["hbmTFLOPS"] == pytest.approx(flops / 2.490368e-6 / 1e12)
    assert p_on["hbmTFLOPS"] == pytest.approx(flops / 3.2768e-6 / 1e12)
    # A and B (1,048,576 B) larger than the MALL: every fetch is a DRAM read again.
    assert p_small["hbmTFLOPS"] == pytest.approx(p_off["hbmTFLOPS"])
    # The compute side is untouched.
    assert p_on["computeTFLOPS"] == pytest.approx(p_off["computeTFLOPS"])
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % (base + ', "mallReuseModel": 1, "mallBytes": 268435456'))
    with pytest.raises(ValueError, match="mallReuseModel 1"):
        RM.Hardware(str(bad))


def test_mall_write_model_drains_cached_c_into_the_mall(tmp_path):
    """mallWriteModel 1 with writes at 4 TB/s to HBM and 8 TB/s into the MALL.
    The last drain of a cached-store row whose A, B and C fit the MALL moves at the
    MALL's rate, shared by the CUs that hold a workgroup: 2048 x 2048 x 128 in
    128x128 tiles fills all 256 CUs, so the drain takes half the cycles; 1024 x 2048
    x 128 holds 128 of them, so each drains at 8 TB/s / 128 against 4 TB/s / 256, a
    quarter of the cycles. The persistent row stores non-temporally and drains to
    HBM as before; so does C larger than the MALL. The DRAM-side time is
    untouched."""
    base = ', "hbmWriteModel": 1, "hbmWriteBytesPerSec": 4e12'
    term = ', "mallWriteModel": 1, "mallWriteBytesPerSec": 8e12, "mallBytes": %d'
    hw = {}
    for name, extra in (("off", ""), ("on", term % (256 << 20)), ("small", term % 1000000)):
        f = tmp_path / (name + ".json")
        f.write_text(_CDNA4_JSON % (base + extra))
        hw[name] = RM.Hardware(str(f))
    row = dict(K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2, regsPerThread=128)
    full, half = dict(M=2048, N=2048, **row), dict(M=1024, N=2048, **row)
    off, on, small = (RM.predict(hw[n], **full) for n in ("off", "on", "small"))
    assert on["tEpilogueCycles"] == pytest.approx(0.5 * off["tEpilogueCycles"])
    assert small["tEpilogueCycles"] == pytest.approx(off["tEpilogueCycles"])
    assert on["hbmTFLOPS"] == pytest.approx(off["hbmTFLOPS"])
    off, on, small = (RM.predict(hw[n], **half) for n in ("off", "on", "small"))
    assert off["totalCtas"] == 128.0
    assert on["tEpilogueCycles"] == pytest.approx(0.25 * off["tEpilogueCycles"])
    assert small["tEpilogueCycles"] == pytest.approx(off["tEpilogueCycles"])
    persistent = dict(full, stages=4, schedule=2)
    assert RM.predict(hw["on"], **persistent)["tEpilogueCycles"] == \
        pytest.approx(RM.predict(hw["off"], **persistent)["tEpilogueCycles"])
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % (term % (256 << 20)))
    with pytest.raises(ValueError, match="mallWriteModel 1"):
        RM.Hardware(str(bad))


def test_fill_latency_model_adds_one_wait_per_round(tmp_path):
    """fillLatencyModel 1 with fillLatencySec 1 us: the prediction's time grows by
    one microsecond per round of one-tile-per-workgroup workgroups (fullWaves)
    and by one for a persistent grid, whatever its tile count."""
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % "")
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % ', "fillLatencyModel": 1, "fillLatencySec": 1e-6')
    hw_off, hw_on = RM.Hardware(str(off)), RM.Hardware(str(on))
    for cfg, rounds in [
        (dict(M=4096, N=4096, K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2, regsPerThread=128), None),
        (dict(M=8192, N=8192, K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=4, regsPerThread=185,
              schedule=2), 1.0),
    ]:
        a, b = RM.predict(hw_off, **cfg), RM.predict(hw_on, **cfg)
        want_rounds = rounds if rounds is not None else math.ceil(a["wavesExact"])
        assert b["fillRounds"] == want_rounds
        flops = 2.0 * cfg["M"] * cfg["N"] * cfg["K"]
        assert b["predictedTFLOPS"] == pytest.approx(flops / (flops / (a["predictedTFLOPS"] * 1e12) +
                                                             want_rounds * 1e-6) / 1e12)
        assert b["predictedTFLOPS"] == pytest.approx(min(b["computeTFLOPS"], b["hbmTFLOPS"]))


def test_persistent_step_model_scales_by_the_skeleton_of_the_class(tmp_path):
    """persistentStepModel 1 on the placeholders (4 cycles per MFMA per CU, one
    blended 128 B/cycle LDS rate). The skeleton rows' own reads + MFMAs:
      128x128x64 w64x64 (4 waves, one per SIMD): tC = 32 MFMAs x 4 waves x 4 =
        512, tS = 4 x (64 + 64) x 64 x 2 B / 128 = 512: 1024 cycles;
      256x128x32 w64x64 (8 waves, two per SIMD): tC = 16 x 8 x 4 = 512,
        tS = 8 x 128 x 32 x 2 / 128 = 512: 1024 cycles.
    With measured K tiles of 768 and 896 cycles the ratios are 0.75 and 0.875.
    A 128x64x64 w64x32 persistent row (one wave per SIMD) has tC = 16 x 4 x 4 =
    256 and tS = 4 x 96 x 64 x 2 / 128 = 384, so 0.75 x 640 = 480 cycles; the
    256x128x32 row itself 0.875 x 1024 = 896. One-tile-per-workgroup rows keep
    their schedule's K-step."""
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % ', "persistentStepModel": 1, "persistentStepCycles1": 768, '
                                '"persistentStepCycles2": 896')
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % "")
    hw_on, hw_off = RM.Hardware(str(on)), RM.Hardware(str(off))
    small = dict(M=8192, N=8192, K=4096, BM=128, BN=64, BK=64, warpM=64, warpN=32, stages=6, regsPerThread=131,
                 groupM=8, schedule=2)
    assert RM.predict(hw_off, **small)["tStepCycles"] == pytest.approx(640.0)
    assert RM.predict(hw_on, **small)["tStepCycles"] == pytest.approx(480.0)
    skel1 = dict(small, BN=128, warpN=64, stages=4, regsPerThread=185)
    assert RM.predict(hw_on, **skel1)["tStepCycles"] == pytest.approx(768.0)
    eight = dict(small, BM=256, BN=128, BK=32, warpM=64, warpN=64, regsPerThread=167, groupM=4)
    assert RM.predict(hw_off, **eight)["tStepCycles"] == pytest.approx(1024.0)
    assert RM.predict(hw_on, **eight)["tStepCycles"] == pytest.approx(896.0)
    uniform = dict(small, schedule=0, stages=3)
    assert RM.predict(hw_on, **uniform)["tStepCycles"] == RM.predict(hw_off, **uniform)["tStepCycles"]
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "persistentStepModel": 1, "persistentStepCycles1": 768')
    with pytest.raises(ValueError, match="persistentStepModel 1"):
        RM.Hardware(str(bad))


def test_ping_pong_step_model_scales_by_the_row_skeleton_of_the_class(tmp_path):
    """pingPongStepModel 1 on the placeholders (4 cycles per MFMA per CU, one
    blended 128 B/cycle LDS rate, four SIMDs). The skeleton rows' own
    max(MFMAs, reads):
      256x256x32 w128x64: tC = 32 MFMAs x 8 waves x 4 = 1024, tS = 8 x (128 + 64)
        x 32 x 2 B / 128 = 768: 1024 cycles;
      256x128x64 w64x64: tC = 32 x 8 x 4 = 1024, tS = 8 x 128 x 64 x 2 / 128 =
        1024: 1024 cycles.
    With measured K tiles of 1100 and 1300 cycles, a BK = 32 ping-pong row's
    K-step is scaled by 1100/1024 and a BK = 64 one's by 1300/1024: 256x256x64
    w128x64 s3 has tC = 64 x 8 x 4 = 2048 and tS = 8 x 192 x 64 x 2 / 128 =
    1536, so 2048 x 1300 / 1024 = 2600. Rows of four waves keep their K-step
    (256x128x64 w128x64: tC = 64 x 4 x 4 = 1024 plus tS = 4 x 192 x 64 x 2 / 128
    = 768, 1792 cycles), and the term needs pingPongModel 1 (the gfx950 preset's
    default)."""
    extra = ', "simdsPerSM": 4, "pingPongModel": 1%s'
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % (extra % ', "pingPongStepModel": 1, "pingPongRowStepCycles1": 1100, '
                                          '"pingPongRowStepCycles2": 1300'))
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % (extra % ""))
    hw_on, hw_off = RM.Hardware(str(on)), RM.Hardware(str(off))
    row = dict(M=8192, N=8192, K=4096, regsPerThread=128, groupM=4)
    for tile, want_off, want_on in (
            (dict(BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=3), 1024.0, 1100.0),
            (dict(BM=256, BN=256, BK=32, warpM=64, warpN=128, stages=4), 1024.0, 1100.0),
            (dict(BM=256, BN=128, BK=64, warpM=64, warpN=64, stages=3), 1024.0, 1300.0),
            (dict(BM=256, BN=256, BK=64, warpM=128, warpN=64, stages=3), 2048.0, 2600.0),
            (dict(BM=256, BN=128, BK=64, warpM=128, warpN=64, stages=3), 1792.0, 1792.0)):
        assert RM.predict(hw_off, **row, **tile)["tStepCycles"] == pytest.approx(want_off)
        assert RM.predict(hw_on, **row, **tile)["tStepCycles"] == pytest.approx(want_on)
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "simdsPerSM": 4, "pingPongModel": 0, "pingPongStepModel": 1, '
                                 '"pingPongRowStepCycles1": 1100, "pingPongRowStepCycles2": 1300')
    with pytest.raises(ValueError, match="pingPongStepModel 1"):
        RM.Hardware(str(bad))


def test_persistent_tile_model_charges_the_epilogue_between_tiles(tmp_path):
    """persistentTileModel 1 on the placeholders, with skeleton K tiles equal to the
    rows' own reads + MFMAs (1024 cycles each, so the step ratio is 1) and
    measured epilogues of 1000 cycles per tile (one compute wave per SIMD) and 500
    (two). At 8192 x 8192 x 128:

      128x128x64 w64x64 s4 (4 compute waves): 16 tiles per slot, body 2 x 1024,
        prologue 2 x 32768 B / 13.0208333 = 5033.1648, drain 2516.5824;
        envelope 32768 / (5033.1648 + 32768 + 16 x 1000 + 2516.5824) = 0.581841
        (without the term 32768 / 40317.7472 = 0.812744);
      256x128x32 w64x64 s6 (8 compute waves): 8 tiles per slot, body 4 x 1024,
        prologue 4 x 24576 B / 13.0208333 = 7549.7472, drain 5033.1648;
        envelope 32768 / (7549.7472 + 32768 + 8 x 500 + 5033.1648) = 0.663980.

    One-tile-per-workgroup rows pay nothing; the term needs the step term."""
    base = ', "persistentStepModel": 1, "persistentStepCycles1": 1024, "persistentStepCycles2": 1024'
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % (base + ', "persistentTileModel": 1, "persistentTileCycles1": 1000, '
                                        '"persistentTileCycles2": 500'))
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % base)
    hw_on, hw_off = RM.Hardware(str(on)), RM.Hardware(str(off))
    four = dict(M=8192, N=8192, K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=4, regsPerThread=185,
                groupM=8, schedule=2)
    assert RM.predict(hw_off, **four)["envelopeEfficiency"] == pytest.approx(32768 / 40317.7472, abs=1e-9)
    p4 = RM.predict(hw_on, **four)
    assert p4["tStepCycles"] == pytest.approx(1024.0) and p4["wavesExact"] == pytest.approx(16.0)
    assert p4["envelopeEfficiency"] == pytest.approx(32768 / (5033.1648 + 32768 + 16000 + 2516.5824), abs=1e-9)
    eight = dict(four, BM=256, BK=32, stages=6, regsPerThread=167, groupM=4)
    p8 = RM.predict(hw_on, **eight)
    assert p8["tStepCycles"] == pytest.approx(1024.0) and p8["wavesExact"] == pytest.approx(8.0)
    assert p8["tPrologueCycles"] == pytest.approx(7549.7472, abs=1e-3)
    assert p8["tEpilogueCycles"] == pytest.approx(5033.1648, abs=1e-3)
    assert p8["envelopeEfficiency"] == pytest.approx(32768 / (7549.7472 + 32768 + 4000 + 5033.1648), abs=1e-9)
    uniform = dict(four, schedule=0)
    assert RM.predict(hw_on, **uniform) == RM.predict(hw_off, **uniform)
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "persistentTileModel": 1, "persistentTileCycles1": 1000, '
                                 '"persistentTileCycles2": 500')
    with pytest.raises(ValueError, match="persistentTileModel 1"):
        RM.Hardware(str(bad))


def test_fill_share_model_fetches_each_panel_slice_once_per_xcd(tmp_path):
    """fillShareModel 1 with HBM at 8 TB/s and the L2s at 8192 B/cycle x 2.4 GHz
    = 19.6608 TB/s, on one XCD. 2048 x 2048 x 1024 on 128x128x64 w64x64 s2: two
    workgroups per CU by LDS (64 KiB rings), so all 256 tiles are resident and the
    XCD holds 16 row and 16 column panels. A K tile of every resident tile is
    256 x 32,768 = 8,388,608 B, of which (16 x 128 + 16 x 128) x 64 x 2 = 524,288 B
    are distinct: 524,288 / 8e12 + 7,864,320 / 19.6608e12 = 0.465536 us against
    8,388,608 / 8e12 = 1.048576 us, a factor 0.443970 on the fill. The fill is
    one tile (stages - 1) of 32,768 B at 8e12 / (2.4e9 x 256) = 13.0208 B/cycle
    per CU, over 2 resident workgroups: 1258.29 cycles, 558.64 with the term."""
    base = ', "numXcds": 1, "l2HitBytesPerCycle": 8192'
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % base)
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % (base + ', "fillShareModel": 1'))
    cfg = dict(M=2048, N=2048, K=1024, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2, regsPerThread=128)
    p_off = RM.predict(RM.Hardware(str(off)), **cfg)
    p_on = RM.predict(RM.Hardware(str(on)), **cfg)
    assert p_off["ctasPerSM"] == 2 and p_off["totalCtas"] == 256
    assert p_off["tPrologueCycles"] == pytest.approx(32768 / (8e12 / (2.4e9 * 256)) / 2)
    factor = (524288 / 8e12 + 7864320 / (8192 * 2.4e9)) / (8388608 / 8e12)
    assert factor == pytest.approx(0.443970, abs=1e-6)
    assert p_on["tPrologueCycles"] == pytest.approx(p_off["tPrologueCycles"] * factor)
    assert p_on["tPrologueCycles"] == pytest.approx(558.64, abs=0.01)
    assert p_on["tEpilogueCycles"] == p_off["tEpilogueCycles"]
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "fillShareModel": 1')
    with pytest.raises(ValueError, match="fillShareModel 1"):
        RM.Hardware(str(bad))


def test_launch_model_adds_the_kernel_boundary_to_each_launch(tmp_path):
    """launchModel 1 with launchOverheadSeconds 2 us: each launch's time grows by
    2 us on both ceilings (a uniform and a persistent row), so the prediction is
    flops / (flops / before + 2 us); a negative overhead is refused."""
    off = tmp_path / "off.json"
    off.write_text(_CDNA4_JSON % "")
    on = tmp_path / "on.json"
    on.write_text(_CDNA4_JSON % ', "launchModel": 1, "launchOverheadSeconds": 2e-6')
    hw_off, hw_on = RM.Hardware(str(off)), RM.Hardware(str(on))
    for cfg in (dict(M=4096, N=4096, K=1024, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2, regsPerThread=128),
                dict(M=8192, N=8192, K=128, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=4, regsPerThread=185,
                     schedule=2)):
        a, b = RM.predict(hw_off, **cfg), RM.predict(hw_on, **cfg)
        flops = 2.0 * cfg["M"] * cfg["N"] * cfg["K"]
        for key in ("predictedTFLOPS", "computeTFLOPS", "hbmTFLOPS"):
            assert b[key] == pytest.approx(flops / (flops / (a[key] * 1e12) + 2e-6) / 1e12)
        assert b["bottleneck"] == a["bottleneck"]
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % ', "launchModel": 1, "launchOverheadSeconds": -1e-6')
    with pytest.raises(ValueError, match="launchModel 1"):
        RM.Hardware(str(bad))


_LABEL_JSON = (', "hbmWriteModel": 1, "hbmWriteBytesPerSec": 5e12, "simdsPerSM": 4, "regsPerSimdLane": 512, '
               '"labelModel": 1, "launchIsolatedSeconds": 3e-6')


def test_label_model_predicts_the_counters_of_one_launch(tmp_path):
    """labelModel 1 on the placeholders (2.4 GHz, 4 cycles per MFMA per CU, HBM
    reads at 8 TB/s, writes at 5 TB/s, one launch from an idle stream costs its
    work plus 3 us):
      duration    = flops / predicted + 3 us;
      DRAM share  = (L2-missed A/B bytes / 8e12 + C bytes / 5e12) / duration;
      MFMA share  = MFMAs (flops / 16384) x 16 cycles / 1024 SIMDs / (duration x 2.4 GHz);
      LDS share   = tiles x K-steps x fragment-read cycles / 256 CUs / (duration x 2.4 GHz);
      body share  = (t(K / 2) - t(K)) / (-t(K) / 2) at K = 4096 (K / 2 holds whole
                    K tiles), from K x 2 at K = 128 on a BK = 128 row (K / 2 does not);
      CU share    = 64 tiles of 128x128 at 1024 x 1024, one round: 64 / 256 = 0.25
                    (and the grid is labelled WAVES, its DRAM share being small)."""
    f = tmp_path / "lab.json"
    f.write_text(_CDNA4_JSON % _LABEL_JSON)
    hw = RM.Hardware(str(f))
    cfg = dict(M=4096, N=4096, K=4096, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=3, regsPerThread=200,
               groupM=4, schedule=1)
    p = RM.predict(hw, **cfg)
    flops = 2.0 * 4096 ** 3
    t = flops / (p["predictedTFLOPS"] * 1e12) + 3e-6
    assert p["kernelSeconds"] == pytest.approx(t)
    assert p["dramWriteBytes"] == 4096 * 4096 * 2
    assert p["dramShare"] == pytest.approx((p["dramReadBytes"] / 8e12 + p["dramWriteBytes"] / 5e12) / t)
    assert p["mfmaShare"] == pytest.approx(flops / 16384 * 16 / 1024 / (t * 2.4e9))
    assert p["ldsShare"] == pytest.approx(p["totalCtas"] * p["kSteps"] * p["tSmemCycles"] / 256 / (t * 2.4e9))
    half = RM.predict(hw, **dict(cfg, K=2048))
    t_half = 2.0 * 4096 * 4096 * 2048 / (half["predictedTFLOPS"] * 1e12) + 3e-6
    assert p["bodyFactor"] == 0.5
    assert p["bodyShare"] == pytest.approx((t_half - t) / (-0.5 * t))
    k128 = dict(M=8192, N=8192, K=128, BM=128, BN=64, BK=128, warpM=64, warpN=32, stages=3, regsPerThread=131,
                groupM=8, schedule=2)
    q = RM.predict(hw, **k128)
    q2 = RM.predict(hw, **dict(k128, K=256))
    tq = 2.0 * 8192 * 8192 * 128 / (q["predictedTFLOPS"] * 1e12) + 3e-6
    tq2 = 2.0 * 8192 * 8192 * 256 / (q2["predictedTFLOPS"] * 1e12) + 3e-6
    assert q["bodyFactor"] == 2.0
    assert q["bodyShare"] == pytest.approx((tq2 - tq) / tq)
    small = RM.predict(hw, M=1024, N=1024, K=4096, BM=128, BN=128, BK=64, warpM=64, warpN=64, stages=2,
                       regsPerThread=128)
    assert small["cuShare"] == pytest.approx(0.25)
    assert small["dramShare"] < 0.70 and small["bottleneck"] == "WAVES"
    # The reference's label without the switch.
    plain = tmp_path / "plain.json"
    plain.write_text(_CDNA4_JSON % _LABEL_JSON.replace('"labelModel": 1', '"labelModel": 0'))
    p0 = RM.predict(RM.Hardware(str(plain)), **cfg)
    assert p0["kernelSeconds"] == 0.0 and p0["predictedTFLOPS"] == p["predictedTFLOPS"]


def test_label_model_is_the_registered_counter_table(mi355x_calibrated):
    """With the committed calibration, the model's label is the label check's
    registered decision table (ridge_amd.labelcheck.counter_label3) applied to the
    model's own predicted counters, on every row of the in-sample sweep, the
    fourth held-out sweep and the BASELINE configs; the first rule that matches
    decides, so a table in another order or with other thresholds disagrees."""
    from ridge_amd import labelcheck as LC
    from ridge_amd import tables as T
    seen = set()
    for name in ("mi355x.csv", "mi355x-heldout4.csv", "mi355x-baseline-configs.csv"):
        for r in T.read(os.path.join(ROOT, "data", "measured", name)).records:
            p = LC.predict_row(mi355x_calibrated, r, True)
            obs = {"dram_share": p["dramShare"], "cu_share": p["cuShare"], "body_share": p["bodyShare"],
                   "lds_share": p["ldsShare"], "mfma_share": p["mfmaShare"]}
            assert LC.counter_label3(obs) == p["bottleneck"], r
            seen.add(p["bottleneck"])
    assert {"HBM", "WAVES", "ENVELOPE", "SMEM", "TENSOR_CORE"} <= seen


def test_label_model_2_counts_busy_shares_at_the_physical_clock(tmp_path):
    """labelModel 2 with powerModel 1 (loadedClockRatio 0.75), clockHz 2.4 GHz and
    nominalClockHz 3.0 GHz: a row whose matrix pipes the power term sees busy a
    share u runs, as the counters count, at 3.0 + (2.4 x 0.75 - 3.0) u GHz, and its
    MFMA and LDS shares are labelModel 1's scaled by (2.4 GHz x powerClockFactor) /
    that clock; the duration, DRAM, body and CU shares are unchanged."""
    base = _LABEL_JSON + ', "powerModel": 1, "loadedClockRatio": 0.75, "nominalClockHz": 3.0e9'
    one, two = tmp_path / "one.json", tmp_path / "two.json"
    one.write_text(_CDNA4_JSON % base)
    two.write_text(_CDNA4_JSON % base.replace('"labelModel": 1', '"labelModel": 2'))
    h1, h2 = RM.Hardware(str(one)), RM.Hardware(str(two))
    for cfg in (dict(M=4096, N=4096, K=4096, BM=256, BN=256, BK=32, warpM=128, warpN=64, stages=3, regsPerThread=200,
                     groupM=4, schedule=1),
                dict(M=4096, N=2048, K=8192, BM=128, BN=256, BK=32, warpM=64, warpN=128, stages=4, regsPerThread=180,
                     groupM=8)):
        a, b = RM.predict(h1, **cfg), RM.predict(h2, **cfg)
        u = a["matrixLoad"]
        assert a["powerClockFactor"] == pytest.approx(1.0 - 0.25 * u)
        clock = 3.0e9 + (2.4e9 * 0.75 - 3.0e9) * u
        assert b["observedClockHz"] == pytest.approx(clock)
        assert a["observedClockHz"] == pytest.approx(2.4e9 * a["powerClockFactor"])
        k = 2.4e9 * a["powerClockFactor"] / clock
        assert b["mfmaShare"] == pytest.approx(a["mfmaShare"] * k)
        assert b["ldsShare"] == pytest.approx(a["ldsShare"] * k)
        for key in ("predictedTFLOPS", "kernelSeconds", "dramShare", "bodyShare", "cuShare"):
            assert b[key] == a[key], key
    bad = tmp_path / "bad.json"
    bad.write_text(_CDNA4_JSON % base.replace('"labelModel": 1', '"labelModel": 2').replace("3.0e9", "2.0e9"))
    with pytest.raises(ValueError, match="labelModel 2"):
        RM.Hardware(str(bad))
