#!/usr/bin/env python3
"""Summaries of rocprofv3 output for the committed profiles.

  rocprof_summary.py stats <run_kernel_stats.csv> [name-substring ...]
      per-kernel call count and average / min / max duration (us)
  rocprof_summary.py counters <pmc-root> <COUNTER> [name-substring ...]
      median KiB per dispatch of each matching kernel in
      <pmc-root>/pmc_<COUNTER>_configs/run_counter_collection.csv
  rocprof_summary.py multi <run_counter_collection.csv> [name-substring ...]
      median per dispatch of every counter of one multi-counter pass, per
      matching kernel
  rocprof_summary.py traffic <pmc-root>
      HBM bytes per dispatch of the GEMV and GEMM kernels (plain and tiled
      GEMM, and the GEMM-tile pack; a workload whose passes are absent is
      skipped) from the two
      counter passes (FETCH_SIZE, WRITE_SIZE; KiB per dispatch), each scaled by
      what the same counter reads for the known-size calibration kernel
      (add_f32 over n = 2^24: 128 MiB read, 64 MiB written per launch).
      <pmc-root> holds pmc_<COUNTER>_<calib|gemv|gemm>/run_counter_collection.csv
      as written by `rocprofv3 --pmc <COUNTER> -f csv -d <pmc-root>/pmc_<COUNTER>_<w>
      -o run -- python3 bench.py --only <w> ...`.  Prints JSON.
"""
from __future__ import annotations

import csv
import json
import os
import statistics
import sys

KERNELS = {
    "gemv_q4_0_q8_0": "gemv_q4_0_q8_0_direct",
    "q8_0_q8_0_gemm": "gemm_wide<false>",
    "q8_0_q8_0_gemm_tiles": "gemm_tiles256_q8",
    "pack_both_to_gemm_tiles": "pack_gemm_tiles_span2",
    "calib": "add_f32_vec4",
}
CALIB_BYTES = {"FETCH_SIZE": 8 << 24, "WRITE_SIZE": 4 << 24}  # per add_f32 launch, n = 2^24


def short_name(name):
    """Kernel name without its parameter list (the last balanced "(...)")."""
    name = name.replace("(anonymous namespace)::", "")
    if name.endswith(")"):
        depth = 0
        for i in range(len(name) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(name[i], 0)
            if depth == 0:
                return name[:i].strip()
    return name


def stats(path, needles):
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Name"]
            if needles and not any(n in name for n in needles):
                continue
            rows.append((name, int(r["Calls"]), float(r["AverageNs"]) / 1e3,
                         float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3))
    for name, calls, avg, mn, mx in rows:
        print(f"| {short_name(name)} | {calls} | {avg:.3f} | {mn:.3f} | {mx:.3f} |")


def counters(root, ctr, needles):
    """Median counter value (KiB) per dispatch of every kernel matching a needle."""
    per = {}
    with open(os.path.join(root, f"pmc_{ctr}_configs", "run_counter_collection.csv")) as f:
        for r in csv.DictReader(f):
            name = short_name(r["Kernel_Name"])
            if needles and not any(n in name for n in needles):
                continue
            key = (name, r["Dispatch_Id"])
            per[key] = per.get(key, 0.0) + float(r["Counter_Value"])
    by = {}
    for (name, _), v in per.items():
        by.setdefault(name, []).append(v)
    for name, vals in sorted(by.items()):
        print(f"| {name} | {ctr} | {len(vals)} | {statistics.median(vals):.1f} |")


def counter_per_dispatch(path, kernel):
    vals = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if kernel in r["Kernel_Name"]:
                key = r["Dispatch_Id"]
                vals[key] = vals.get(key, 0.0) + float(r["Counter_Value"])
    if not vals:
        raise SystemExit(f"{path}: no dispatch of {kernel}")
    v = list(vals.values())
    return statistics.median(v), len(v)


def multi(path, needles):
    per = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if needles and not any(n in name for n in needles):
                continue
            key = (name.split("(")[0], r["Counter_Name"])
            d = per.setdefault(key, {})
            d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    print("| kernel | counter | dispatches | median per dispatch |")
    print("|---|---|---|---|")
    for (kernel, ctr), d in sorted(per.items()):
        print(f"| {kernel} | {ctr} | {len(d)} | {statistics.median(d.values()):.4e} |")


def traffic(root):
    out = {"method": "median KiB per dispatch x 1024, scaled by calib bytes / calib counter"}
    scale = {}
    for ctr, known in CALIB_BYTES.items():
        kib, n = counter_per_dispatch(
            os.path.join(root, f"pmc_{ctr}_calib", "run_counter_collection.csv"), KERNELS["calib"])
        scale[ctr] = known / (kib * 1024.0)
        out[f"calib_{ctr}"] = {"KiB_per_dispatch": kib, "dispatches": n, "known_bytes": known,
                               "scale": scale[ctr]}
    for key, tag in (("gemv_q4_0_q8_0", "gemv"), ("q8_0_q8_0_gemm", "gemm"),
                     ("q8_0_q8_0_gemm_tiles", "gemm"), ("pack_both_to_gemm_tiles", "gemm")):
        if not all(os.path.isdir(os.path.join(root, f"pmc_{ctr}_{tag}")) for ctr in CALIB_BYTES):
            continue  # that workload's counter passes were not run
        total = 0.0
        entry = {"kernel": KERNELS[key]}
        for ctr in CALIB_BYTES:
            kib, n = counter_per_dispatch(
                os.path.join(root, f"pmc_{ctr}_{tag}", "run_counter_collection.csv"), KERNELS[key])
            b = kib * 1024.0 * scale[ctr]
            entry[ctr] = {"KiB_per_dispatch": kib, "dispatches": n, "bytes_scaled": round(b)}
            total += b
        entry["bytes"] = round(total)
        out[key] = entry
    print(json.dumps(out, indent=1))


def main():
    if len(sys.argv) >= 3 and sys.argv[1] == "stats":
        stats(sys.argv[2], sys.argv[3:])
    elif len(sys.argv) == 3 and sys.argv[1] == "traffic":
        traffic(sys.argv[2])
    elif len(sys.argv) >= 3 and sys.argv[1] == "multi":
        multi(sys.argv[2], sys.argv[3:])
    elif len(sys.argv) >= 4 and sys.argv[1] == "counters":
        counters(sys.argv[2], sys.argv[3], sys.argv[4:])
    else:
        print(__doc__)
        sys.exit(2)


if __name__ == "__main__":
    main()
