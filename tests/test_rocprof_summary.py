"""The rocprofv3 summary helpers on synthetic CSVs with known answers (CPU)."""
import csv

from tt_symbiote_amd import rocprof_summary as rs

TRACE_FIELDS = ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"]
COUNTER_FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(tmp_path, dispatches, window=150_000.0):
    """dispatches: (name, duration ns, clock GHz, MFMA busy cycles); GRBM_GUI_ACTIVE is the
    window plus 8 XCDs x clock x duration, split over two rows as per-XCD instances are."""
    tr, ct = tmp_path / "t.csv", tmp_path / "c.csv"
    with open(tr, "w", newline="") as f, open(ct, "w", newline="") as g:
        wt = csv.DictWriter(f, TRACE_FIELDS)
        wc = csv.DictWriter(g, COUNTER_FIELDS)
        wt.writeheader()
        wc.writeheader()
        t = 0
        for i, (name, dur, ghz, busy) in enumerate(dispatches):
            wt.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Start_Timestamp": t,
                         "End_Timestamp": t + dur})
            t += dur + 1000
            grbm = window + 8 * ghz * dur
            for half in (0.25, 0.75):
                wc.writerow({"Dispatch_Id": i, "Kernel_Name": name,
                             "Counter_Name": "GRBM_GUI_ACTIVE", "Counter_Value": grbm * half})
            wc.writerow({"Dispatch_Id": i, "Kernel_Name": name,
                         "Counter_Name": "SQ_VALU_MFMA_BUSY_CYCLES", "Counter_Value": busy})
    return str(tr), str(ct)


def test_clock_window_fit_and_mfma_fraction(tmp_path, capsys):
    # memory kernels at 2.3 GHz of several lengths fix the window; an MFMA kernel at 2.0 GHz
    # whose busy cycles fill half of its SIMD cycles at that clock
    mem = [("copy_kernel", d, 2.3, 0.0) for d in (5_000, 20_000, 80_000, 160_000)]
    dur = 400_000
    busy = 0.5 * 1024 * 2.0 * dur      # SIMDs x clock (cycles per ns) x duration
    tr, ct = _write(tmp_path, mem + [("gemm_kernel", dur, 2.0, busy)])
    table = rs._dispatch_table(tr, ct)
    a, b = rs.profiler_window_cycles(table)
    assert abs(a - 150_000.0) < 1e-3 * 150_000 and abs(b / 8 - 2.3) < 1e-6
    flops = 1.0e12
    rs.clock_report(tr, ct, ["gemm"], {"gemm_kernel": flops})
    line = [ln for ln in capsys.readouterr().out.splitlines() if "gemm_kernel" in ln][0].split()
    ghz, executed_frac_at_clk = float(line[2]), float(line[6])
    assert abs(ghz - 2.0) < 1e-3
    # the published 2.5 PFLOP/s is 1017 flops per SIMD cycle at 2.4 GHz, the MFMA's 1024 is
    # 0.7% above it
    assert abs(executed_frac_at_clk - 0.5 * 1024 * 1024 * 2.4e9 / 2.5e15) < 1e-3
    # algorithmic: 1e12 flops in 400 us = 2.5 PFLOP/s, i.e. 1.0 of the 2.4 GHz peak and
    # 2.4 / 2.0 of the peak at 2.0 GHz
    assert abs(float(line[8]) - 1.0) < 2e-3 and abs(float(line[9]) - 1.2) < 2e-3
