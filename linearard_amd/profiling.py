"""Summaries of rocprofv3 CSV output for the measurement files under profiles/.

Two summaries, both printed as text the repository keeps:

* ``stats``: per-kernel launch count and average / total duration from a
  ``--kernel-trace --stats`` run (``*_kernel_stats.csv``).
* ``traffic``: HBM bytes per launch of each library kernel from two
  ``--pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE`` runs (``*_counter_collection.csv``)
  of ``bench.py --copy-calibration MIB``.  The derived counters are scaled by
  what they read for the calibration dispatch (``torch.neg`` over MIB MiB of
  float32: exactly MIB MiB read and MIB MiB written), so the result is in
  bytes whatever the counters' own unit or coverage.  The JSON it prints is
  what ``bench.py`` reads from ``profiles/traffic_<config>.json``.

    python -m linearard_amd.profiling stats RUN_kernel_stats.csv
    python -m linearard_amd.profiling traffic --fetch F.csv --write W.csv --calib-mib 1024 --config cfg4
"""

from __future__ import annotations

import argparse
import collections
import csv
import json
import sys

# kernel-name fragment -> timing-hook kernel id (include/linearard_amd.h)
KERNEL_NAMES = {
    "hot_fwd_kernel": "forward",
    "fused_fwd_kernel": "forward",
    "hot_dq_kernel": "row_grad",
    "hot_bwd_kernel": "col_grad",
    "logits_kl_forward_kernel": "logits_forward",
    "logits_kl_grad_kernel": "logits_grad",
}
CALIBRATION_FRAGMENT = "neg_kernel"


def kernel_id(name: str):
    for frag, kid in KERNEL_NAMES.items():
        if frag in name:
            return kid
    return None


def stats_table(path: str, top: int = 12) -> str:
    rows = list(csv.DictReader(open(path, newline="")))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    out = [f"{'kernel':64s} {'calls':>6s} {'avg ms':>10s} {'total ms':>10s} {'share':>7s}"]
    for r in rows[:top]:
        out.append(f"{r['Name'][:64]:64s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e6:10.3f} "
                   f"{float(r['TotalDurationNs']) / 1e6:10.3f} {float(r['Percentage']):6.1f}%")
    return "\n".join(out)


def counter_means(path: str, counter: str):
    """Mean counter value per dispatch, by kernel name (instances of one dispatch summed)."""
    per_dispatch = collections.defaultdict(float)
    names = {}
    for r in csv.DictReader(open(path, newline="")):
        if r["Counter_Name"] != counter:
            continue
        key = r["Dispatch_Id"]
        per_dispatch[key] += float(r["Counter_Value"])
        names[key] = r["Kernel_Name"]
    by_name = collections.defaultdict(list)
    for key, v in per_dispatch.items():
        by_name[names[key]].append(v)
    return {n: sum(v) / len(v) for n, v in by_name.items()}


def traffic(fetch_csv: str, write_csv: str, calib_mib: int, config: str) -> dict:
    fetch = counter_means(fetch_csv, "FETCH_SIZE")
    write = counter_means(write_csv, "WRITE_SIZE")
    calib_bytes = calib_mib << 20

    def calibration(table, what):
        vals = [v for n, v in table.items() if CALIBRATION_FRAGMENT in n]
        if not vals:
            raise SystemExit(f"no calibration dispatch ({CALIBRATION_FRAGMENT}) in the {what} run")
        return calib_bytes / vals[0]

    f_fetch = calibration(fetch, "FETCH_SIZE")
    f_write = calibration(write, "WRITE_SIZE")
    out = {"config": config, "calibration_bytes": calib_bytes,
           "scale_fetch_bytes_per_count": f_fetch, "scale_write_bytes_per_count": f_write,
           "raw_fetch_size": {}, "raw_write_size": {}, "bytes_per_launch": {}, "read_bytes": {}, "write_bytes": {}}
    for name in sorted(set(fetch) | set(write)):
        kid = kernel_id(name)
        if kid is None:
            continue
        rf, rw = fetch.get(name, 0.0), write.get(name, 0.0)
        out["raw_fetch_size"][kid] = rf
        out["raw_write_size"][kid] = rw
        out["read_bytes"][kid] = rf * f_fetch
        out["write_bytes"][kid] = rw * f_write
        out["bytes_per_launch"][kid] = rf * f_fetch + rw * f_write
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--calib-mib", type=int, required=True)
    t.add_argument("--config", default="cfg4")
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print(stats_table(a.csv))
    else:
        json.dump(traffic(a.fetch, a.write, a.calib_mib, a.config), sys.stdout, indent=1)
        print()


if __name__ == "__main__":
    main()
