"""Summaries of rocprofv3 CSV output (--output-format csv) for the text files kept under profiles/.

  python -m gwenedeg_amd.profsum stats DIR [--top N]
      the kernel statistics (--kernel-trace --stats: *_kernel_stats.csv under DIR) as a markdown table
  python -m gwenedeg_amd.profsum traffic FETCH_DIR WRITE_DIR --kernel REGEX [--calib REGEX] [--calib-bytes B]
                                 [--algo-bytes A] [--json OUT]
      HBM bytes per dispatch of the kernels matching REGEX from two counter runs (--pmc FETCH_SIZE, --pmc WRITE_SIZE:
      *_counter_collection.csv), each counter scaled by what it reads for the calibration kernel (a kernel of known
      traffic: CALIB_BYTES read and CALIB_BYTES written), against A algorithmic bytes per dispatch
  python -m gwenedeg_amd.profsum busy DIR [DIR ...] --kernel REGEX [--cus 256] [--ses 32]
      per kernel matching REGEX: the mean per dispatch of every counter in the runs (SQ_* summed over their instances,
      GRBM_* the largest instance), and rocprofv3's derived metrics where their counters are there:
      MfmaUtil = 100 SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs), VALUBusy = 100 SQ_ACTIVE_INST_VALU / CUs /
      GRBM_GUI_ACTIVE (SQ_ACTIVE_INST_VALU: quad-cycles summed over the SIMDs of each shader engine); and the same
      normalised by the cycles the kernel's waves were present (SQ_BUSY_CYCLES, summed over the --ses shader engines,
      each with 4 x CUs / SEs SIMDs), which counter collection does not dilute as it does GRBM_GUI_ACTIVE:
      valu_issue = 4 SQ_INSTS_VALU / (SIMDs x busy), valu_active = 4 SQ_ACTIVE_INST_VALU / (SIMDs x busy),
      mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x busy), busy = SQ_BUSY_CYCLES / SEs
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys


def _rows(d: str, suffix: str):
    files = sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    for f in files:
        with open(f, newline="") as fh:
            yield from csv.DictReader(fh)


def _col(row: dict, *names):
    low = {k.lower(): k for k in row}
    for n in names:
        if n.lower() in low:
            return row[low[n.lower()]]
    raise KeyError(f"none of {names} in {list(row)}")


def stats(d: str, top: int = 25) -> str:
    rows = []
    for r in _rows(d, "kernel_stats.csv"):
        rows.append((_col(r, "Name", "KernelName"), int(_col(r, "Calls")), float(_col(r, "TotalDurationNs")),
                     float(_col(r, "AverageNs")), float(_col(r, "MinNs")), float(_col(r, "MaxNs"))))
    rows.sort(key=lambda r: -r[2])
    tot = sum(r[2] for r in rows)
    out = ["| kernel | calls | avg us | min us | max us | total ms | share |", "|---|---:|---:|---:|---:|---:|---:|"]
    for n, calls, t, avg, mn, mx in rows[:top]:
        n = re.sub(r"\(.*$", "", n)[:90]
        out.append(f"| `{n}` | {calls} | {avg / 1e3:.2f} | {mn / 1e3:.2f} | {mx / 1e3:.2f} | {t / 1e6:.3f} | "
                   f"{100 * t / tot:.1f}% |")
    return "\n".join(out)


def _counter(d: str, name: str):
    """{dispatch id: (kernel name, counter value summed over its instances)}"""
    acc = {}
    for r in _rows(d, "counter_collection.csv"):
        if _col(r, "Counter_Name") != name:
            continue
        k = _col(r, "Dispatch_Id")
        kn = _col(r, "Kernel_Name")
        v = float(_col(r, "Counter_Value"))
        acc[k] = (kn, acc.get(k, (kn, 0.0))[1] + v)
    return acc


def traffic(fetch_dir, write_dir, kernel, calib="neg_kernel", calib_bytes=1 << 30, algo_bytes=None):
    res = {}
    for cname, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        acc = _counter(d, cname)
        cal = [v for kn, v in acc.values() if re.search(calib, kn)]
        if not cal:
            raise SystemExit(f"no calibration dispatch ({calib}) in {d}")
        factor = calib_bytes / max(cal)  # bytes per counter unit
        vals = {}
        for kn, v in acc.values():
            if re.search(kernel, kn):
                vals.setdefault(re.sub(r"\(.*$", "", kn), []).append(v * factor)
        res[cname] = {"calib_reading": max(cal), "bytes_per_unit": factor,
                      "per_kernel": {k: {"dispatches": len(v), "mean_bytes": sum(v) / len(v)} for k, v in vals.items()}}
    n = sum(x["dispatches"] for x in res["FETCH_SIZE"]["per_kernel"].values())
    fetch = sum(x["dispatches"] * x["mean_bytes"] for x in res["FETCH_SIZE"]["per_kernel"].values()) / n
    nw = sum(x["dispatches"] for x in res["WRITE_SIZE"]["per_kernel"].values())
    write = sum(x["dispatches"] * x["mean_bytes"] for x in res["WRITE_SIZE"]["per_kernel"].values()) / nw
    out = {"kernel": kernel, "dispatches": n, "fetch_bytes_per_launch": round(fetch), "write_bytes_per_launch": round(write),
           "traffic_bytes_per_launch": round(fetch + write), "counters": res}
    if algo_bytes:
        out["algorithmic_bytes_per_launch"] = algo_bytes
        out["traffic_over_algorithmic"] = round((fetch + write) / algo_bytes, 4)
    return out


def busy(dirs, kernel, cus=256, ses=32):
    per = {}  # kernel -> counter -> {dispatch: value}
    for d in dirs:
        for r in _rows(d, "counter_collection.csv"):
            kn = re.sub(r"\(.*$", "", _col(r, "Kernel_Name"))
            if not re.search(kernel, kn):
                continue
            c, disp, v = _col(r, "Counter_Name"), (d, _col(r, "Dispatch_Id")), float(_col(r, "Counter_Value"))
            slot = per.setdefault(kn, {}).setdefault(c, {})
            slot[disp] = max(slot.get(disp, 0.0), v) if c.startswith("GRBM_") else slot.get(disp, 0.0) + v
    out = {}
    for kn, cs in per.items():
        mean = {c: sum(v.values()) / len(v) for c, v in cs.items()}
        o = {"dispatches": max(len(v) for v in cs.values()), "mean_per_dispatch": {c: round(x, 1) for c, x in mean.items()}}
        g = mean.get("GRBM_GUI_ACTIVE")
        if g and "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
            o["MfmaUtil_pct"] = round(100 * mean["SQ_VALU_MFMA_BUSY_CYCLES"] / (g * 4 * cus), 2)
        if g and "SQ_ACTIVE_INST_VALU" in mean:
            o["VALUBusy_pct"] = round(100 * mean["SQ_ACTIVE_INST_VALU"] / cus / g, 2)
        if mean.get("SQ_INSTS_MFMA") and "SQ_INSTS_VALU" in mean:
            o["valu_insts_per_mfma"] = round(mean["SQ_INSTS_VALU"] / mean["SQ_INSTS_MFMA"], 3)
        b = mean.get("SQ_BUSY_CYCLES")
        if b:
            simd_cycles = 4 * cus * b / ses  # (every SIMD over the cycles one shader engine had waves)
            o["busy_cycles_per_se"] = round(b / ses)
            for key, c, f in (("valu_issue_pct", "SQ_INSTS_VALU", 4), ("valu_active_pct", "SQ_ACTIVE_INST_VALU", 4),
                              ("mfma_busy_pct", "SQ_VALU_MFMA_BUSY_CYCLES", 1)):
                if c in mean:
                    o[key] = round(100 * f * mean[c] / simd_cycles, 2)
        out[kn] = o
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a1 = sub.add_parser("stats")
    a1.add_argument("dir")
    a1.add_argument("--top", type=int, default=25)
    a2 = sub.add_parser("traffic")
    a2.add_argument("fetch_dir")
    a2.add_argument("write_dir")
    a2.add_argument("--kernel", required=True)
    a2.add_argument("--calib", default="neg_kernel")
    a2.add_argument("--calib-bytes", type=float, default=float(1 << 30))
    a2.add_argument("--algo-bytes", type=float, default=None)
    a2.add_argument("--json", default=None)
    a3 = sub.add_parser("busy")
    a3.add_argument("dirs", nargs="+")
    a3.add_argument("--kernel", required=True)
    a3.add_argument("--cus", type=int, default=256)
    a3.add_argument("--ses", type=int, default=32)
    a = ap.parse_args(argv)
    if a.cmd == "busy":
        print(json.dumps(busy(a.dirs, a.kernel, a.cus, a.ses), indent=1))
        return
    if a.cmd == "stats":
        print(stats(a.dir, a.top))
        return
    out = traffic(a.fetch_dir, a.write_dir, a.kernel, a.calib, a.calib_bytes, a.algo_bytes)
    text = json.dumps(out, indent=1)
    if a.json:
        with open(a.json, "w") as fh:
            fh.write(text + "\n")
    print(text)


if __name__ == "__main__":
    sys.exit(main())
