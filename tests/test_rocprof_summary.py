"""The counter summary behind roofline.traffic: calibration by the copy of
known size, last dispatch per kernel, kernel-name normalisation."""
import csv
import importlib

rs = importlib.import_module("mtp-glora_amd.rocprof_summary")

FIELDS = ["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for i, (name, grid, val) in enumerate(rows):
            w.writerow(dict(Dispatch_Id=i + 1, Grid_Size=grid, Kernel_Name=name, Counter_Name=counter,
                            Counter_Value=val))


def test_traffic_calibration_and_last_dispatch(tmp_path):
    f, w = tmp_path / "f.csv", tmp_path / "w.csv"
    copy = "kv_copy_rows_kernel"
    fwd = "_ZN3mga15attn_fwd_kernelILi1ELi128EDF16bEEvNS_8AttnArgsE"
    # prefix fill (small copy), calibration (largest grid), attention, commit
    _write(f, "FETCH_SIZE", [(copy, 100, 50.0), (copy, 1000, 512.0), (fwd, 10, 300.0), (copy, 80, 40.0)])
    _write(w, "WRITE_SIZE", [(copy, 100, 100.0), (copy, 1000, 1024.0), (fwd, 10, 10.0), (copy, 80, 80.0)])
    r = rs.traffic(str(f), str(w), calib_read=1024 * 1024, calib_write=1024 * 1024, config=2)
    assert r["FETCH_SIZE_calibration"]["factor"] == 2.0
    assert r["WRITE_SIZE_calibration"]["factor"] == 1.0
    assert r["kernels"]["attn_fwd_kernel"] == {"fetch_bytes": 600 * 1024, "write_bytes": 10 * 1024,
                                               "traffic_bytes": 610 * 1024}
    # the commit (last dispatch), not the prefix fill
    assert r["kernels"][copy]["fetch_bytes"] == 80 * 1024


def test_kernel_base_names():
    assert rs.kernel_base("_ZN3mga18attn_bwd_dq_kernelILi128EDF16bEEvNS_8AttnArgsE") == "attn_bwd_dq_kernel"
    assert rs.kernel_base("void mga::attn_fwd_kernel<1, 128, float>(mga::AttnArgs)") == "attn_fwd_kernel"
    assert rs.kernel_base("kv_copy_rows_kernel") == "kv_copy_rows_kernel"


def test_forward_launches_of_one_call_are_summed(tmp_path):
    """The forward's 4-wave launch and its two-group tail launch are one call:
    traffic and counters add over the last run of consecutive forward
    dispatches; an earlier forward call is not counted, nor is any other
    kernel's earlier dispatch."""
    f, w = tmp_path / "f.csv", tmp_path / "w.csv"
    copy = "kv_copy_rows_kernel"
    f1 = "_ZN3mga15attn_fwd_kernelILi128EDF16bLi1EEEvNS_8AttnArgsEii"
    f2 = "_ZN3mga15attn_fwd_kernelILi128EDF16bLi2EEEvNS_8AttnArgsEii"
    _write(f, "FETCH_SIZE", [(copy, 1000, 512.0), (f1, 10, 7.0), (f2, 5, 9.0), (copy, 80, 40.0),
                             (f1, 10, 300.0), (f2, 5, 20.0)])
    _write(w, "WRITE_SIZE", [(copy, 1000, 1024.0), (f1, 10, 1.0), (f2, 5, 1.0), (copy, 80, 80.0),
                             (f1, 10, 8.0), (f2, 5, 2.0)])
    r = rs.traffic(str(f), str(w), calib_read=1024 * 1024, calib_write=1024 * 1024, config=2)
    assert r["kernels"]["attn_fwd_kernel"]["fetch_bytes"] == 2 * 320 * 1024
    assert r["kernels"]["attn_fwd_kernel"]["write_bytes"] == 10 * 1024
    assert r["kernels"][copy]["fetch_bytes"] == 80 * 1024
    c = tmp_path / "c.csv"
    with open(c, "w", newline="") as fh:
        wr = csv.DictWriter(fh, fieldnames=FIELDS)
        wr.writeheader()
        for d, (name, util, gui, busy) in enumerate([(f1, 40.0, 300.0, 10.0), (f2, 20.0, 100.0, 3.0)]):
            for cn, v in (("MfmaUtil", util), ("GRBM_GUI_ACTIVE", gui), ("SQ_VALU_MFMA_BUSY_CYCLES", busy)):
                wr.writerow(dict(Dispatch_Id=d + 1, Grid_Size=1, Kernel_Name=name, Counter_Name=cn,
                                 Counter_Value=v))
    got = rs.counters_by_kernel([str(c)])["attn_fwd_kernel"]
    assert got["GRBM_GUI_ACTIVE"] == 400.0 and got["SQ_VALU_MFMA_BUSY_CYCLES"] == 13.0
    assert got["MfmaUtil"] == (40.0 * 300.0 + 20.0 * 100.0) / 400.0


def test_kernel_labels_tell_the_forward_forms_apart():
    assert rs.kernel_label("_ZN3mga15attn_fwd_kernelILi128EDF16bLi2EEEvNS_8AttnArgsEii") == \
        "attn_fwd_kernel (two-group)"
    assert rs.kernel_label("_ZN3mga15attn_fwd_kernelILi128EDF16bLi1EEEvNS_8AttnArgsEii") == \
        "attn_fwd_kernel (8-wave pair)"
    assert rs.kernel_label("_ZN3mga15attn_fwd_kernelILi64EDF16_Li0EEEvNS_8AttnArgsEii") == \
        "attn_fwd_kernel (4-wave)"
    assert rs.kernel_label("attn_fwd_kernel") == "attn_fwd_kernel"
    assert rs.kernel_label("void mga::attn_fwd_kernel<128, __bf16, 2>(mga::AttnArgs, int, int)") == \
        "attn_fwd_kernel (two-group)"
    assert rs.kernel_label("_ZN3mga18attn_bwd_dq_kernelILi128EDF16bEEvNS_8AttnArgsE") == "attn_bwd_dq_kernel"
    assert rs.kernel_label("_ZN3mga18attn_bwd_dq_kernelILi128EDF16bLi1EEEvNS_8AttnArgsEii") == \
        "attn_bwd_dq_kernel (8-wave pair)"
    assert rs.kernel_label("_ZN3mga18attn_bwd_dq_kernelILi64EDF16_Li2EEEvNS_8AttnArgsEii") == \
        "attn_bwd_dq_kernel (two-group)"
    assert rs.kernel_label("void mga::attn_bwd_dq_kernel<128, __bf16, 0>(mga::AttnArgs, int, int)") == \
        "attn_bwd_dq_kernel (4-wave)"


def test_kernel_clocks_from_gui_active_over_duration(tmp_path):
    """Clock = GRBM_GUI_ACTIVE summed over 8 XCDs / 8 over the traced
    duration; dispatches without the counter and other kernels are left out."""
    c, t = tmp_path / "c.csv", tmp_path / "t.csv"
    dq = "_ZN3mga18attn_bwd_dq_kernelILi128EDF16bLi1EEEvNS_8AttnArgsEii"
    with open(c, "w", newline="") as fh:
        wr = csv.DictWriter(fh, fieldnames=FIELDS)
        wr.writeheader()
        # 8 XCDs x 250 000 cycles over 100 us: 2.5 GHz; 8 x 200 000 over 100 us: 2.0 GHz
        for d, v in ((1, 250000.0), (2, 200000.0), (3, 200000.0)):
            for x in range(8):
                wr.writerow(dict(Dispatch_Id=d, Grid_Size=1, Kernel_Name=dq, Counter_Name="GRBM_GUI_ACTIVE",
                                 Counter_Value=v))
    with open(t, "w", newline="") as fh:
        wr = csv.DictWriter(fh, fieldnames=["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        wr.writeheader()
        wr.writerow(dict(Dispatch_Id=1, Kernel_Name=dq, Start_Timestamp=0, End_Timestamp=100000))
        wr.writerow(dict(Dispatch_Id=2, Kernel_Name=dq, Start_Timestamp=0, End_Timestamp=100000))
        wr.writerow(dict(Dispatch_Id=3, Kernel_Name="kv_copy_rows_kernel", Start_Timestamp=0, End_Timestamp=1000))
        wr.writerow(dict(Dispatch_Id=4, Kernel_Name=dq, Start_Timestamp=0, End_Timestamp=5000))
    r = rs.kernel_clocks(str(c), str(t))
    assert list(r) == ["attn_bwd_dq_kernel"]
    assert r["attn_bwd_dq_kernel"]["dispatches"] == 2
    assert r["attn_bwd_dq_kernel"]["min_ghz"] == 2.0 and r["attn_bwd_dq_kernel"]["max_ghz"] == 2.5
    assert r["attn_bwd_dq_kernel"]["median_us"] == 100.0
