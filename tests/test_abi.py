"""The C ABI library loads and exports every declared symbol, and the variant
table is self-consistent. No GPU calls."""
import ctypes
import glob
import os
import re

import pytest

from ridge_amd import gemm as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ridge_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(glob.glob(os.path.join(ROOT, "include", "*.h"))))
def test_every_declared_symbol_is_exported(header):
    names = _declared(header)
    assert names, header
    from ridge_amd import model as RM
    libs = {
        "ridge_gemm.h": G.LIB_PATH,
        "ridge_model.h": RM.LIB_PATH,
    }
    path = libs.get(os.path.basename(header))
    if path is None:
        pytest.skip("no library mapped for %s" % header)
    L = ctypes.CDLL(path)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_table_has_24_registered_rows_with_consistent_fields():
    vs = G.variants()
    assert len(vs) == 24
    keys = [v.key() for v in vs]
    assert len(set(keys)) == 24
    for v in vs:
        assert v.BM in (64, 128, 256) and v.BN in (64, 128, 256) and v.BK in (32, 64, 128)
        compute_waves = (v.BM // v.WM) * (v.BN // v.WN)
        ring = v.stages * (v.BM * v.BK + v.BK * v.BN) * 2
        assert v.schedule in (0, 1, 2)
        assert v.pingPong == (1 if v.schedule == 1 else 0)
        if v.schedule == 2:
            # Persistent: two loader wavefronts; LDS = ring + a 16-row-multiple
            # staging region per compute wavefront.
            assert 2 <= v.stages <= 8
            assert v.waves == compute_waves + 2
            staging = v.ldsBytes - ring
            assert staging > 0 and staging % (compute_waves * 16 * v.WN * 2) == 0
        else:
            assert 2 <= v.stages <= 5
            assert v.waves == compute_waves
            assert v.ldsBytes == ring
            assert v.schedule == (1 if v.waves == 8 and v.stages >= 3 else 0)
        assert v.threads == 64 * v.waves
        assert v.ldsBytes <= 160 * 1024
        assert v.regsPerThread == v.vgprs + v.agprs and v.regsPerThread > 0
        assert v.occupancy >= 1
        assert G.find_variant(*v.key()) == v.index
    assert G.find_variant(512, 512, 128, 64, 64, 8, 8) == -1


def test_no_variant_spills():
    # The reference refuses spilling kernels as ground truth (setup-box.sh:96-104).
    assert [v.label() for v in G.variants() if v.scratchBytes != 0] == []


def test_divisibility_and_bad_launches_are_rejected_before_any_gpu_call():
    i = G.find_variant(256, 256, 32, 128, 64, 4, 4)
    v = G.variant(i)
    assert v.divides(4096, 4096, 4096)
    assert not v.divides(4096, 4096, 4016)
    assert not v.divides(128, 4096, 4096)
    assert not v.divides(0, 256, 64)
    L = G.lib()
    # Non-dividing shape, null pointers, misaligned pointers and a bad index all
    # return hipErrorInvalidValue without touching a device.
    assert L.ridge_gemm_launch(i, 4096, 4096, 4096, 4096, 4096, 4016, None) == G.HIP_ERROR_INVALID_VALUE
    assert L.ridge_gemm_launch(i, None, 4096, 4096, 256, 256, 64, None) == G.HIP_ERROR_INVALID_VALUE
    assert L.ridge_gemm_launch(i, 4098, 4096, 4096, 256, 256, 64, None) == G.HIP_ERROR_INVALID_VALUE
    assert L.ridge_gemm_launch(999, 4096, 4096, 4096, 256, 256, 64, None) == G.HIP_ERROR_INVALID_VALUE
    with pytest.raises(IndexError):
        G.variant(24)


def test_offset_guard_admits_up_to_2_pow_31_and_refuses_beyond():
    """In-kernel byte offsets into an A or B tile are 32-bit: a shape is admitted
    only while BM * K and BK * N stay below 2^31."""
    for v in G.variants():
        k_max = (0x7FFFFFFF // v.BM) // v.BK * v.BK
        assert v.divides(v.BM, v.BN, k_max), v.label()
        assert not v.divides(v.BM, v.BN, k_max + v.BK), v.label()
        n_max = (0x7FFFFFFF // v.BK) // v.BN * v.BN
        assert v.divides(v.BM, n_max, v.BK), v.label()
        assert not v.divides(v.BM, n_max + v.BN, v.BK), v.label()


def test_gemm_refuses_bad_operands_before_any_launch():
    import torch
    a = torch.zeros((256, 64), dtype=torch.float16)
    b = torch.zeros((64, 256), dtype=torch.float16)
    with pytest.raises(G.RidgeGemmError, match="float16"):
        G.gemm(a.float(), b)
    with pytest.raises(G.RidgeGemmError, match="device tensors"):
        G.gemm(a, b)


def test_ridge_check_lists_the_variant_table_without_a_gpu():
    import subprocess
    exe = os.path.join(ROOT, "ridge_amd", "bin", "ridge-check")
    out = subprocess.run([exe, "--list-variants"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    assert out.stdout == G.variant_table_csv()
    bad = subprocess.run([exe, "--no-such-option"], capture_output=True, text=True, timeout=60)
    assert bad.returncode == 2 and "unknown option" in bad.stderr


def test_variant_table_csv():
    text = G.variant_table_csv()
    lines = text.strip().splitlines()
    assert lines[0].startswith("idx,BM,BN,BK,WM,WN,stages,groupM,ldsBytes,threads,regsPerThread")
    assert len(lines) == 25
    assert lines[0].endswith(",pingPong,schedule")
    for i in (0, len(lines) - 2):
        row = lines[i + 1].split(",")
        v = G.variant(i)
        assert [int(x) for x in row[:11]] == [i, v.BM, v.BN, v.BK, v.WM, v.WN, v.stages, v.groupM, v.ldsBytes,
                                              v.threads, v.regsPerThread]
        assert int(row[-1]) == v.schedule
    assert sum(1 for l in lines[1:] if l.endswith(",2")) == sum(1 for v in G.variants() if v.schedule == 2) >= 1


def test_persistent_rows_are_labelled():
    ps = [v for v in G.variants() if v.schedule == 2]
    assert ps and all(v.label().endswith(" persistent") and v.schedule_name == "persistent" for v in ps)
    assert all(not v.label().endswith("persistent") for v in G.variants() if v.schedule != 2)


def test_binding_struct_layouts_match_the_libraries():
    """The ctypes stubs declare the C structs themselves; each library reports its
    own sizeof, and loading refuses a disagreement (a short struct would be
    overwritten past its end by the library)."""
    from ridge_amd import model as RM
    assert G.lib().ridge_gemm_variant_struct_size() == ctypes.sizeof(G._VariantStruct)
    L = RM.lib()
    assert L.ridge_model_config_size() == ctypes.sizeof(RM._Config)
    assert L.ridge_model_prediction_size() == ctypes.sizeof(RM._Prediction)
    # The prediction ends with the gfx950 fields, after the reference's, and the
    # counter observables last.
    assert [f for f, _ in RM._Prediction._fields_][-18:] == ["tailClockFactor", "l2HitBytes", "powerClockFactor",
                                                             "fillRounds", "refillMissShare", "mallLoad",
                                                             "mallStretch", "kernelSeconds", "dramReadBytes",
                                                             "dramWriteBytes", "dramShare", "bodyFactor",
                                                             "bodyShare", "cuShare", "mfmaShare", "ldsShare",
                                                             "matrixLoad", "observedClockHz"]


def test_bound_callables_hold_their_operands_and_refuse_a_closed_handle():
    """A bound launch keeps the objects whose raw pointers it converted alive for
    as long as it exists (no GPU call is made here), and a bound or direct
    hipBLASLt call on a closed handle is refused before reaching the library."""
    import gc
    import weakref

    class Operand:
        def data_ptr(self):
            return 0

    a = Operand()
    ref = weakref.ref(a)
    call = G.bound_launch(0, a, Operand(), Operand(), 256, 256, 64, stream=0)
    del a
    gc.collect()
    assert ref() is not None
    del call
    gc.collect()
    assert ref() is None
    closed = G.BlasLt.__new__(G.BlasLt)
    closed._h = None
    with pytest.raises(G.RidgeGemmError, match="closed"):
        closed.bound_gemm(Operand(), Operand(), Operand(), 256, 256, 64, stream=0)
    with pytest.raises(G.RidgeGemmError, match="closed"):
        closed.gemm(Operand(), Operand(), Operand(), 256, 256, 64, stream=0)


def test_row_split_plans_whole_rounds_and_refuses_before_any_launch():
    """The body row 256x256x32 s3 holds one workgroup per CU (96 KiB of LDS), so on
    256 CUs a split gives it the rows of whole rounds of 256 tiles, in whole row
    panels: 6144 x 3072 (24 x 12 = 288 tiles) -> 21 panels = 5376 rows (252 tiles);
    12288 x 1536 (48 x 6) -> 42 panels; 12288 x 3072 (576 tiles) -> 504 tiles, 42
    panels. A grid of whole rounds keeps all its rows (M), one below a round none;
    on 192 CUs 4096^3 (16 x 16 tiles) gets 12 panels. Every refusal comes back
    before a launch (fake, aligned pointers; no GPU is touched)."""
    body = G.find_variant(256, 256, 32, 128, 64, 3, 4)
    tail = G.find_variant(128, 128, 64, 64, 64, 4, 8)
    assert G.split_rows(body, 6144, 3072, 6144) == 5376
    assert G.split_rows(body, 12288, 1536, 6144) == 10752
    assert G.split_rows(body, 12288, 3072, 3072) == 10752
    assert G.split_rows(body, 4096, 4096, 4096) == 4096
    assert G.split_rows(body, 4096, 4096, 4096, num_cus=192) == 3072
    assert G.split_rows(body, 3072, 1536, 3072) == 0
    assert G.split_rows(body, 6000, 3072, 6144) == -1 and G.split_rows(-1, 6144, 3072, 6144) == -1
    assert G.split_rows(body, 6144, 3072, 6144, num_cus=0) == -1
    ok = (16, 32, 48)
    cases = [(body, tail, 0, ok), (body, tail, 6144, ok), (body, tail, 5300, ok), (body, tail, 5376, (16, 32, 50)),
             (body, tail, 5376, (0, 32, 48)), (body, -1, 5376, ok), (-1, tail, 5376, ok)]
    for b, t, rows, ptrs in cases:
        assert G.launch_split(b, t, rows, *ptrs, 6144, 3072, 6144, 0) == 1, (b, t, rows, ptrs)
