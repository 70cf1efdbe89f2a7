"""Summaries of rocprofv3 output for the attention kernels (CSV output format).

  python -m sdxl_hip.profiling stats <dir> [--last N] kernel-trace stats (per-kernel avg duration;
                                                      --last N: over each kernel's last N dispatches)
  python -m sdxl_hip.profiling counters <dir> [name]  mean PMC counter value per dispatch of a kernel
  python -m sdxl_hip.profiling traffic --kernel NAME --fetch DIR --write DIR
                                       --copy-fetch DIR --copy-write DIR --copy-mib N
      HBM bytes per launch of NAME from FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled
      by what the same counter reads for a device copy of N MiB (read N MiB, write N MiB).
  python -m sdxl_hip.profiling report LABEL=DIR_A,DIR_B,KERNEL ...
      one markdown row per LABEL from two counter passes (PASS_A / PASS_B below) over the
      dispatches whose name contains KERNEL: MFMA
      utilisation and per-MFMA instruction and stall ratios (see report_row).
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
from collections import defaultdict


def _rows(root: str, suffix: str):
    for f in sorted(glob.glob(os.path.join(root, "**", f"*{suffix}"), recursive=True)):
        with open(f) as fh:
            yield from csv.DictReader(fh)


def kernel_stats(root: str, last: int = 0):
    """{kernel: (calls, avg_ns, total_ns)} from *kernel_stats.csv (or *kernel_trace.csv); with
    last > 0, from the trace over each kernel's last `last` dispatches (in start order)."""
    out = {}
    if last > 0:
        acc = defaultdict(list)
        for r in _rows(root, "kernel_trace.csv"):
            acc[r["Kernel_Name"]].append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
        for k, v in acc.items():
            d = [e - s for s, e in sorted(v)[-last:]]
            out[k] = (len(d), sum(d) / len(d), float(sum(d)))
        return out
    for r in _rows(root, "kernel_stats.csv"):
        out[r["Name"]] = (int(r["Calls"]), float(r["AverageNs"]), float(r["TotalDurationNs"]))
    if not out:
        acc = defaultdict(list)
        for r in _rows(root, "kernel_trace.csv"):
            acc[r["Kernel_Name"]].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        out = {k: (len(v), sum(v) / len(v), float(sum(v))) for k, v in acc.items()}
    return out


def counters(root: str, kernel_substr: str = ""):
    """{counter: mean value per dispatch} over dispatches whose kernel name contains kernel_substr.
    Values of one dispatch are summed over instances first (rocprofv3 may emit one row per XCD)."""
    per_dispatch = defaultdict(lambda: defaultdict(float))
    for r in _rows(root, "counter_collection.csv"):
        if kernel_substr and kernel_substr not in r.get("Kernel_Name", ""):
            continue
        per_dispatch[r["Counter_Name"]][r.get("Dispatch_Id", "0")] += float(r["Counter_Value"])
    return {k: sum(v.values()) / len(v) for k, v in per_dispatch.items() if v}


def traffic(kernel: str, fetch_dir: str, write_dir: str, copy_fetch: str, copy_write: str, copy_mib: float):
    copy_bytes = copy_mib * (1 << 20)
    f_k = counters(fetch_dir, kernel)["FETCH_SIZE"] * 1024.0
    w_k = counters(write_dir, kernel)["WRITE_SIZE"] * 1024.0
    f_c = counters(copy_fetch, "")["FETCH_SIZE"] * 1024.0
    w_c = counters(copy_write, "")["WRITE_SIZE"] * 1024.0
    f_scale = copy_bytes / f_c
    w_scale = copy_bytes / w_c
    return {"fetch_bytes_raw": f_k, "write_bytes_raw": w_k, "fetch_scale": f_scale, "write_scale": w_scale,
            "fetch_bytes": f_k * f_scale, "write_bytes": w_k * w_scale,
            "traffic_bytes": f_k * f_scale + w_k * w_scale}


PASS_A = ("MfmaUtil", "SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_ACTIVE_INST_VALU", "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES",
          "SQ_WAIT_INST_LDS", "SQ_VALU_MFMA_COEXEC_CYCLES")
PASS_B = ("SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_VALU_CVT", "SQ_INSTS_LDS", "SQ_LDS_IDX_ACTIVE", "SQ_LDS_BANK_CONFLICT",
          "SQ_ACTIVE_INST_LDS", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "GRBM_GUI_ACTIVE")
REPORT_HEADER = ("| kernel / workload | MfmaUtil % | MFMA / dispatch | VALU instr / MFMA | exp / MFMA | cvt / MFMA | "
                 "VALU-active cycles / MFMA | LDS instr / MFMA | LDS bank-conflict % | wave time waiting on s_waitcnt % | "
                 "wave time waiting to issue % |\n|---|---|---|---|---|---|---|---|---|---|---|")


def report_row(label: str, dir_a: str, dir_b: str, kernel: str) -> str:
    """Per-MFMA ratios of one kernel. Counter semantics used: SQ_INSTS_* count wave instructions
    (SQ_INSTS_VALU includes the MFMAs); SQ_ACTIVE_INST_VALU, SQ_WAVE_CYCLES and SQ_WAIT_* count in
    units of 4 shader clocks; MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE (max over
    XCDs) * SIMDs) in percent, as rocprofv3 derives it."""
    a, b = counters(dir_a, kernel), counters(dir_b, kernel)
    mfma = a["SQ_INSTS_MFMA"]
    valu = a["SQ_INSTS_VALU"] - mfma
    waves = a["SQ_WAVE_CYCLES"]
    conflict = 100.0 * b["SQ_LDS_BANK_CONFLICT"] / max(b["SQ_LDS_IDX_ACTIVE"], 1.0)
    return (f"| {label} | {a['MfmaUtil']:.1f} | {mfma:.0f} | {valu / mfma:.2f} | "
            f"{b['SQ_INSTS_VALU_TRANS_F32'] / mfma:.2f} | {b['SQ_INSTS_VALU_CVT'] / mfma:.2f} | "
            f"{4.0 * a['SQ_ACTIVE_INST_VALU'] / mfma:.1f} | {b['SQ_INSTS_LDS'] / mfma:.2f} | {conflict:.1f} | "
            f"{100.0 * b['SQ_WAIT_ANY'] / waves:.0f} | {100.0 * b['SQ_WAIT_INST_ANY'] / waves:.0f} |")


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("stats")
    a.add_argument("dir")
    a.add_argument("--last", type=int, default=0)
    b = sub.add_parser("counters")
    b.add_argument("dir")
    b.add_argument("name", nargs="?", default="")
    c = sub.add_parser("traffic")
    for k in ("kernel", "fetch", "write", "copy_fetch", "copy_write"):
        c.add_argument("--" + k.replace("_", "-"), required=True)
    c.add_argument("--copy-mib", type=float, required=True)
    r = sub.add_parser("report")
    r.add_argument("rows", nargs="+", help="LABEL=PASS_A_DIR,PASS_B_DIR,KERNEL_SUBSTRING")
    args = ap.parse_args()
    if args.cmd == "stats":
        for name, (calls, avg, tot) in sorted(kernel_stats(args.dir, args.last).items(), key=lambda x: -x[1][2]):
            print(f"{avg / 1e3:10.2f} us avg  {calls:6d} calls  {tot / 1e6:9.3f} ms total  {name[:110]}")
    elif args.cmd == "counters":
        for k, v in sorted(counters(args.dir, args.name).items()):
            print(f"{k:32s} {v:18.1f}")
    elif args.cmd == "report":
        print(REPORT_HEADER)
        for row in args.rows:
            label, dirs = row.split("=", 1)
            da, db, kernel = dirs.split(",")
            print(report_row(label, da, db, kernel))
    else:
        t = traffic(args.kernel, args.fetch, args.write, args.copy_fetch, args.copy_write, args.copy_mib)
        for k, v in t.items():
            print(f"{k}: {v:.6g}")


if __name__ == "__main__":
    main()
