"""Summaries of rocprofv3 CSV output (--output-format csv) for the text files kept under profiles/.

  python -m gwenedeg_amd.profsum stats DIR [--top N]
      the kernel statistics (--kernel-trace --stats: *_kernel_stats.csv under DIR) as a markdown table
  python -m gwenedeg_amd.profsum traffic FETCH_DIR WRITE_DIR --kernel REGEX [--calib REGEX] [--calib-bytes B]
                                 [--algo-bytes A] [--json OUT]
      HBM bytes per dispatch of the kernels matching REGEX from two counter runs (--pmc FETCH_SIZE, --pmc WRITE_SIZE:
      *_counter_collection.csv), each counter scaled by what it reads for the calibration kernel (a kernel of known
      traffic: CALIB_BYTES read and CALIB_BYTES written), against A algorithmic bytes per dispatch
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
    a = ap.parse_args(argv)
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
