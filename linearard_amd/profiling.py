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

* ``counters``: per library kernel, the mean of every counter per dispatch
  over any number of ``--pmc`` passes (``*_counter_collection.csv``, one pass
  per file), the dispatch duration from the same records, and the derived
  figures the design quotes (clock, MFMA-pipe busy, wave-time fractions,
  instructions per wave), each with its formula in the printed notes.

    python -m linearard_amd.profiling stats RUN_kernel_stats.csv
    python -m linearard_amd.profiling traffic --fetch F.csv --write W.csv --calib-mib 1024 --config cfg4
    python -m linearard_amd.profiling counters P1.csv P2.csv P3.csv
"""

from __future__ import annotations

import argparse
import collections
import csv
import json
import sys

# kernel-name fragment -> kernel id (the timing hook's, include/linearard_amd.h,
# for the throughput and logits kernels)
KERNEL_NAMES = {
    "hot_fwdq_kernel": "forward_rowgrad",
    "hot_fwdq_batch_kernel": "forward_rowgrad",
    "hot_fwd_kernel": "forward",
    "fused_fwd_kernel": "forward",
    "hot_dq_kernel": "row_grad",
    "hot_bwd_kernel": "col_grad",
    "logits_kl_forward_kernel": "logits_forward",
    "logits_kl_grad_kernel": "logits_grad",
    # the stage entry points' kernels (no timing-hook id: profile names only)
    "row_kernel<0,": "stage_a_lse",
    "row_kernel<1,": "stage_b_kl",
    "row_kernel<2,": "stage_c_dq",
    "col_kernel<": "stage_c_dk",
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


# MI355X: 8 XCDs, 32 CUs per XCD, 4 SIMDs per CU, 4 shader engines per XCD.
XCDS, CUS, SIMDS, SES = 8, 256, 1024, 32
KERNEL_ORDER = ("forward", "forward_rowgrad", "row_grad", "col_grad", "logits_forward", "logits_grad",
                "stage_a_lse", "stage_b_kl", "stage_c_dq", "stage_c_dk")


def counter_table(paths) -> dict:
    """{kernel id: {"duration_ms": mean dispatch duration, "dispatches": n,
    counter: mean value per dispatch}} over the given pass files."""
    out = {}
    for path in paths:
        per = collections.defaultdict(dict)  # (kid, dispatch) -> {counter: summed value}
        dur = {}
        for r in csv.DictReader(open(path, newline="")):
            kid = kernel_id(r["Kernel_Name"])
            if kid is None:
                continue
            key = (kid, r["Dispatch_Id"])
            per[key][r["Counter_Name"]] = per[key].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            dur[key] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-6
        by_kid = collections.defaultdict(list)
        for key, vals in per.items():
            by_kid[key[0]].append((dur[key], vals))
        for kid, recs in by_kid.items():
            d = out.setdefault(kid, {"duration_ms": [], "dispatches": 0})
            d["duration_ms"] += [r[0] for r in recs]
            d["dispatches"] = max(d["dispatches"], len(recs))
            for name in recs[0][1]:
                if name == "GRBM_GUI_ACTIVE":  # in every pass: keep it per pass for the clock of that pass
                    d.setdefault("_grbm", []).extend((r[1][name], r[0]) for r in recs)
                    continue
                d[name] = sum(r[1][name] for r in recs) / len(recs)
    for d in out.values():
        durs = d.pop("duration_ms")
        d["duration_ms"] = sum(durs) / len(durs)
        grbm = d.pop("_grbm", [])
        if grbm:
            d["GRBM_GUI_ACTIVE"] = sum(g for g, _ in grbm) / len(grbm)
            d["clock_ghz"] = sum(g / XCDS / (t * 1e-3) for g, t in grbm) / len(grbm) / 1e9
    return out


def derived(d: dict) -> dict:
    """Figures derived from one kernel's counter means (formulas in COUNTER_NOTES)."""
    out = {}
    cyc = d.get("clock_ghz", 0) * 1e9 * d["duration_ms"] * 1e-3  # shader cycles per dispatch
    if cyc and "SQ_VALU_MFMA_BUSY_CYCLES" in d:
        out["mfma_busy"] = d["SQ_VALU_MFMA_BUSY_CYCLES"] / (SIMDS * cyc)
    if "SQ_VALU_MFMA_BUSY_CYCLES" in d and d.get("SQ_INSTS_MFMA"):
        out["mfma_cycles_per_inst"] = d["SQ_VALU_MFMA_BUSY_CYCLES"] / d["SQ_INSTS_MFMA"]
    if cyc and "SQ_BUSY_CYCLES" in d:
        out["sq_busy"] = d["SQ_BUSY_CYCLES"] / (SES * cyc)
    wc = d.get("SQ_WAVE_CYCLES")
    for c, k in (("SQ_ACTIVE_INST_ANY", "wave_active_any"), ("SQ_ACTIVE_INST_VALU", "wave_active_valu"),
                 ("SQ_ACTIVE_INST_LDS", "wave_active_lds"), ("SQ_WAIT_ANY", "wave_wait_any"),
                 ("SQ_WAIT_INST_ANY", "wave_wait_inst_any"), ("SQ_WAIT_INST_LDS", "wave_wait_inst_lds"),
                 ("SQ_VALU_MFMA_COEXEC_CYCLES", "mfma_coexec_per_wave_cycle")):
        if wc and c in d:
            out[k] = d[c] / wc
    if d.get("SQ_INSTS_MFMA"):
        m = d["SQ_INSTS_MFMA"]
        for c, k in (("SQ_INSTS_VALU", "valu_per_mfma"), ("SQ_INSTS_VALU_TRANS_F32", "trans_per_mfma"),
                     ("SQ_INSTS_LDS", "lds_per_mfma"), ("SQ_INSTS_SALU", "salu_per_mfma")):
            if c in d:
                out[k] = d[c] / m
    return out


COUNTER_NOTES = """\
Derived figures (counters summed over the whole GPU per dispatch):
- clock_ghz = GRBM_GUI_ACTIVE / 8 XCDs / dispatch duration (the average shader clock under counters)
- mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x clock x duration): share of SIMD cycles the matrix pipe is busy
- mfma_cycles_per_inst = SQ_VALU_MFMA_BUSY_CYCLES / SQ_INSTS_MFMA (32 for v_mfma_f32_32x32x16)
- sq_busy = SQ_BUSY_CYCLES / (32 shader engines x clock x duration)
- wave_* = the named SQ counter / SQ_WAVE_CYCLES: share of the waves' resident time (both in the same unit)
- *_per_mfma = instruction counts per MFMA instruction (the kernels issue a fixed number of MFMAs per 32x32 sub-block)
"""


def counters_report(paths) -> str:
    tab = counter_table(paths)
    kids = [k for k in KERNEL_ORDER if k in tab]
    names = sorted({n for k in kids for n in tab[k] if n.isupper() or n.startswith("SQ_") or n.startswith("GRBM")})
    lines = ["| counter (mean per dispatch) | " + " | ".join(kids) + " |", "|---|" + "---|" * len(kids)]
    lines.append("| dispatches | " + " | ".join(str(tab[k]["dispatches"]) for k in kids) + " |")
    lines.append("| duration ms | " + " | ".join(f"{tab[k]['duration_ms']:.3f}" for k in kids) + " |")
    for n in names:
        lines.append(f"| {n} | " + " | ".join(f"{tab[k].get(n, float('nan')):.4g}" for k in kids) + " |")
    der = {k: derived(tab[k]) for k in kids}
    lines += ["", "| derived | " + " | ".join(kids) + " |", "|---|" + "---|" * len(kids)]
    lines.append("| clock_ghz | " + " | ".join(f"{tab[k].get('clock_ghz', float('nan')):.3f}" for k in kids) + " |")
    for n in sorted({n for k in kids for n in der[k]}):
        lines.append(f"| {n} | " + " | ".join(f"{der[k].get(n, float('nan')):.3f}" for k in kids) + " |")
    return "\n".join(lines) + "\n\n" + COUNTER_NOTES


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
    c = sub.add_parser("counters")
    c.add_argument("csv", nargs="+")
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print(stats_table(a.csv))
    elif a.cmd == "counters":
        print(counters_report(a.csv))
    else:
        json.dump(traffic(a.fetch, a.write, a.calib_mib, a.config), sys.stdout, indent=1)
        print()


if __name__ == "__main__":
    main()
