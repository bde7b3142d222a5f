"""linearard_amd.profiling: the rocprofv3 CSV summaries behind profiles/
(kernel stats table, counter traffic scaled by a plain copy of known size)."""

import csv

from linearard_amd import profiling as P


def _write(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def _counters(path, counter, per_kernel):
    """Counter CSV with two instances (XCD rows) per dispatch and two dispatches per kernel."""
    rows = []
    disp = 0
    for name, value in per_kernel.items():
        for _ in range(2):
            disp += 1
            rows.append([disp, name, counter, value * 0.25])
            rows.append([disp, name, counter, value * 0.75])
    _write(path, ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"], rows)


def test_traffic_scales_by_the_copy_calibration(tmp_path):
    mib = 64
    nbytes = mib << 20
    fetch, write = tmp_path / "f.csv", tmp_path / "w.csv"
    # the copy reads and writes nbytes; the counters count 2048 B and 1024 B units
    _counters(fetch, "FETCH_SIZE", {"void at::native::neg_kernel_impl": nbytes / 2048,
                                    "void lard::hot_bwd_kernel<128, true>(lard::HotArgs)": 1000.0,
                                    "void lard::hot_fwd_kernel<128, true>(lard::HotArgs)": 10.0})
    _counters(write, "WRITE_SIZE", {"void at::native::neg_kernel_impl": nbytes / 1024,
                                    "void lard::hot_bwd_kernel<128, true>(lard::HotArgs)": 500.0})
    t = P.traffic(str(fetch), str(write), mib, "cfgX")
    assert t["config"] == "cfgX" and t["calibration_bytes"] == nbytes
    assert abs(t["scale_fetch_bytes_per_count"] - 2048) < 1e-9
    assert abs(t["scale_write_bytes_per_count"] - 1024) < 1e-9
    assert t["read_bytes"]["col_grad"] == 1000.0 * 2048 and t["write_bytes"]["col_grad"] == 500.0 * 1024
    assert t["bytes_per_launch"]["col_grad"] == 1000.0 * 2048 + 500.0 * 1024
    assert t["bytes_per_launch"]["forward"] == 10.0 * 2048  # no WRITE_SIZE row: zero writes
    assert "neg" not in " ".join(t["bytes_per_launch"])  # the calibration copy is not a library kernel


def test_stats_table_sorts_by_total_time(tmp_path):
    path = tmp_path / "s.csv"
    _write(path, ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage"],
           [["small", 2, 2e6, 1e6, 10.0], ["big", 4, 18e6, 4.5e6, 90.0]])
    lines = P.stats_table(str(path)).splitlines()
    assert lines[1].startswith("big") and lines[2].startswith("small")
    assert "4.500" in lines[1] and "90.0%" in lines[1]


def test_counter_summary_means_clock_and_mfma_busy(tmp_path):
    """Two passes, two dispatches of one kernel each, every counter split over
    two instance rows: the summary sums instances, averages dispatches, takes
    durations from the timestamps, and derives the clock and MFMA-pipe share."""
    header = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    name = "void lard::hot_dq_kernel<128, true>(lard::HotArgs)"
    ms, ghz = 2.0, 2.0
    cycles = ms * 1e-3 * ghz * 1e9

    def pass_rows(counters, first):
        rows = []
        for disp in (first, first + 1):
            for c, v in counters.items():
                rows += [[disp, name, c, v / 2, 1000, 1000 + int(ms * 1e6)]] * 2
        return rows

    p1, p2 = tmp_path / "p1.csv", tmp_path / "p2.csv"
    _write(p1, header, pass_rows({"GRBM_GUI_ACTIVE": 8 * cycles, "SQ_INSTS_MFMA": 1e6,
                                  "SQ_VALU_MFMA_BUSY_CYCLES": 0.5 * 1024 * cycles}, 1))
    _write(p2, header, pass_rows({"GRBM_GUI_ACTIVE": 8 * cycles, "SQ_WAVE_CYCLES": 4e8, "SQ_WAIT_INST_ANY": 1e8}, 9))
    tab = P.counter_table([str(p1), str(p2)])
    d = tab["row_grad"]
    assert d["dispatches"] == 2 and abs(d["duration_ms"] - ms) < 1e-9
    assert abs(d["clock_ghz"] - ghz) < 1e-9 and d["SQ_INSTS_MFMA"] == 1e6
    der = P.derived(d)
    assert abs(der["mfma_busy"] - 0.5) < 1e-9
    assert abs(der["mfma_cycles_per_inst"] - 0.5 * 1024 * cycles / 1e6) < 1e-6
    assert abs(der["wave_wait_inst_any"] - 0.25) < 1e-12
    text = P.counters_report([str(p1), str(p2)])
    assert "| row_grad |" in text and "mfma_busy" in text and "clock_ghz" in text
