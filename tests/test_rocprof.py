"""CPU tests of the rocprofv3 CSV readers and the per-phase summary."""
import csv

from ridge_amd import rocprof as R

OURS = "_Z14gemmMfmaKernelILi64ELi64ELi64ELi32ELi32ELi4ELi8EEvPKDF16_S2_PDF16_iiii"
FILL = "_Z17fillUniformKernelPDF16_my"


def _write_trace(path, names_and_ns):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        t = 1000
        for i, (name, ns) in enumerate(names_and_ns):
            w.writerow(["KERNEL_DISPATCH", i + 1, name, t, t + ns])
            t += ns + 10


def _write_counters(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for r in rows:
            w.writerow(r)


def test_short_names_mangled_and_demangled():
    assert R.short_name(OURS) == "gemmMfmaKernel"
    assert R.short_name(FILL) == "fillUniformKernel"
    assert R.short_name("void gemmMfmaPingPongKernel<256, 256, 32>(half const*)") == "gemmMfmaPingPongKernel"
    assert R.short_name("void ridge::gemmMfmaKernel<64, 64>(half const*)") == "gemmMfmaKernel"
    # Truncated mangled names do not index past their end.
    assert R.short_name("_Z3") == "_Z3"
    assert R.short_name("_Z10abc") == "_Z10abc"
    assert R.short_name("Cijk_Ailk_Bljk_HHS_BH_MT256x256x64") == "Cijk_Ailk_Bljk_HHS_BH_MT256x256x64"


def test_phases_split_at_every_change_of_kernel(tmp_path):
    seq = [(OURS, 6000)] * 5 + [(FILL, 100)] * 2 + [(OURS, 8000)] * 4 + [(FILL, 100)]
    _write_trace(tmp_path / "run_kernel_trace.csv", seq)
    rows = R.trace_table(R.parse_trace_dir(str(tmp_path)), min_run=1)
    assert [(r["kernel"], r["launches"]) for r in rows] == [
        ("gemmMfmaKernel", 5), ("fillUniformKernel", 2), ("gemmMfmaKernel", 4), ("fillUniformKernel", 1)]
    assert rows[0]["median_us"] == 6.0 and rows[2]["median_us"] == 8.0
    kept = R.trace_table(R.parse_trace_dir(str(tmp_path)), min_run=3)
    assert [r["launches"] for r in kept] == [5, 4]


def test_counters_sum_instances_and_take_grbm_per_xcd(tmp_path):
    rows = []
    for d in (1, 2, 3):
        # FETCH_SIZE reported per instance (summed), GRBM_GUI_ACTIVE per XCD (max).
        rows += [[d, OURS, "FETCH_SIZE", 100.0 * d], [d, OURS, "FETCH_SIZE", 50.0]]
        rows += [[d, OURS, "GRBM_GUI_ACTIVE", 1000.0 + x] for x in range(8)]
    _write_counters(tmp_path / "run_counter_collection.csv", rows)
    (row,) = R.counter_table(R.parse_counter_dir(str(tmp_path)), min_run=1)
    assert row["launches"] == 3
    assert row["FETCH_SIZE"] == 250.0  # median of 150, 250, 350
    assert row["fetch_bytes"] == 250.0 * R.FETCH_SCALE * 1024
    assert row["GRBM_GUI_ACTIVE"] == 1007.0
