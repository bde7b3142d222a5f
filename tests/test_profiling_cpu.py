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
