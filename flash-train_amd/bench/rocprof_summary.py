#!/usr/bin/env python3
"""Summarises rocprofv3 runs of bench.py into a profiles/*.md page and a
profiles/traffic.json entry.

Expected layout under --dir (rocprofv3 ... --output-format csv -d <dir>/<pass> -o run):
  kt/run_kernel_trace.csv, kt/run_kernel_stats.csv, kt.log   kernel trace + the bench JSON line
  F/run_counter_collection.csv                               --pmc FETCH_SIZE
  W/run_counter_collection.csv                               --pmc WRITE_SIZE
  M/run_counter_collection.csv                               --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_LDS_BANK_CONFLICT
                                                                   SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE
and under --copy the same F / W passes of `bench.py --copy-calibration`.

The kernel duration reported is the mean over the bench run's timed dispatches
only (the last `steps` dispatches of the kernel in the trace; warm-up
dispatches excluded), next to the bench's own HIP-event time per step.

  python flash-train_amd/bench/rocprof_summary.py --dir gpurun_out/p_square_8192 --copy gpurun_out/p_copy \\
      --kernel mfma16_gemm --title mfma16_gemm_256x256 --workload square_8192 \\
      --bench-args "--workload square_8192" --out profiles/mfma16_gemm_256x256_square_8192.md
"""

from __future__ import annotations

import argparse
import collections
import csv
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
FP32_PEAK = 157.3
HALF_PEAK = 2500.0  # dense bf16 / fp16 MFMA, TFLOP/s
PEAK_CLOCK_HZ = 2.4e9  # MI355X highest shader clock (the peaks above are quoted at it)


def rows(path: str) -> list:
    with open(path) as f:
        return list(csv.DictReader(f))


def counters(path: str, match: str) -> dict:
    agg = collections.defaultdict(list)
    for r in rows(path):
        if match in r["Kernel_Name"]:
            agg[r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in agg.items()}


def bench_json(log: str) -> dict:
    with open(log) as f:
        lines = [l for l in f if l.startswith("{")]
    return json.loads(lines[-1])


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--dir", required=True)
    ap.add_argument("--copy", required=True)
    ap.add_argument("--kernel", required=True, help="substring of the dominant kernel's name")
    ap.add_argument("--title", required=True)
    ap.add_argument("--workload", required=True, help="traffic.json key")
    ap.add_argument("--bench-args", required=True)
    ap.add_argument("--out", required=True)
    a = ap.parse_args()

    bj = bench_json(os.path.join(a.dir, "kt.log"))
    steps, warmup = bj["steps"], bj["warmup"]
    trace = [r for r in rows(os.path.join(a.dir, "kt", "run_kernel_trace.csv")) if a.kernel in r["Kernel_Name"]]
    trace.sort(key=lambda r: int(r["Start_Timestamp"]))
    durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in trace]  # us
    timed = durs[-steps:]
    kernel_us = sum(timed) / len(timed)
    others = collections.defaultdict(list)
    for r in rows(os.path.join(a.dir, "kt", "run_kernel_trace.csv")):
        others[r["Kernel_Name"]].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)

    cfg = bj["config"]
    m, n, k = cfg["m"], cfg["n"], cfg["k"]
    flops = 2.0 * m * n * k
    half = bj.get("dtype") in ("bf16", "fp16")
    peak = HALF_PEAK if half else FP32_PEAK
    # A grouped launch (bench.py --grouped E) reads one k x n weight per expert.
    experts = cfg.get("experts", 1)
    alg = (2.0 if half else 4.0) * (m * k + experts * k * n) + 4.0 * m * n * (2 if cfg.get("c") else 1)
    fetch = counters(os.path.join(a.dir, "F", "run_counter_collection.csv"), a.kernel)["FETCH_SIZE"]
    write = counters(os.path.join(a.dir, "W", "run_counter_collection.csv"), a.kernel)["WRITE_SIZE"]
    mc = counters(os.path.join(a.dir, "M", "run_counter_collection.csv"), a.kernel)
    cf = counters(os.path.join(a.copy, "F", "run_counter_collection.csv"), "copyBuffer")["FETCH_SIZE"]
    cw = counters(os.path.join(a.copy, "W", "run_counter_collection.csv"), "copyBuffer")["WRITE_SIZE"]
    fs, ws = 262144.0 / cf, 262144.0 / cw  # the calibration copy moves 256 MiB each way
    traffic = fetch * 1024 * fs + write * 1024 * ws
    busy = mc["SQ_VALU_MFMA_BUSY_CYCLES"] / (1024.0 * mc["GRBM_GUI_ACTIVE"] / 8.0)
    # MFMA cycles per SIMD over the traced kernel time at the highest shader clock: a lower bound on
    # the busy fraction whatever the clock was.  GRBM_GUI_ACTIVE spans the counter window, which
    # adds several microseconds to a dispatch (a 4-5 us reduction kernel reads as a 6 GHz clock),
    # so the ratio above understates short kernels.
    busy_floor = mc["SQ_VALU_MFMA_BUSY_CYCLES"] / 1024.0 / (kernel_us * 1e-6 * PEAK_CLOCK_HZ)
    conflict = mc["SQ_LDS_BANK_CONFLICT"] / mc["SQ_LDS_IDX_ACTIVE"] if mc.get("SQ_LDS_IDX_ACTIVE") else 0.0

    b = "python3 bench.py --no-cpu --no-overhead --no-configs " + a.bench_args
    d = a.dir
    lines = [
        f"# `{a.title}` on `{a.workload}`", "",
        "Commands, run from the repository root on the MI355X box after "
        "`cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT`, then the summary:", "", "```",
        f"rocprofv3 --kernel-trace --stats --output-format csv -d {d}/kt -o run -- {b} > {d}/kt.log",
        f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d {d}/F -o run -- {b} --steps 3 --warmup 1 --warm-ms 0",
        f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d {d}/W -o run -- {b} --steps 3 --warmup 1 --warm-ms 0",
        f"rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE GRBM_GUI_ACTIVE "
        f"--output-format csv -d {d}/M -o run -- {b} --steps 3 --warmup 1 --warm-ms 0",
        f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d {a.copy}/F -o run -- python3 bench.py --copy-calibration",
        f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d {a.copy}/W -o run -- python3 bench.py --copy-calibration",
        f"python3 flash-train_amd/bench/rocprof_summary.py --dir {d} --copy {a.copy} --kernel {a.kernel} "
        f"--title {a.title} --workload {a.workload} --bench-args \"{a.bench_args}\" --out {a.out}",
        "```", "",
        f"## Kernel time per timed step ({steps} timed dispatches after {warmup} warm-up, from `run_kernel_trace.csv`)", "",
        "| Kernel | Dispatches in trace | Mean µs, timed steps | Min µs | Max µs |", "|---|---:|---:|---:|---:|",
    ]
    for name, ds in sorted(others.items(), key=lambda kv: -sum(kv[1])):
        t = ds[-steps:]
        lines.append(f"| `{name[:120]}` | {len(ds)} | {sum(t) / len(t):.1f} | {min(t):.1f} | {max(t):.1f} |")
    step_us = bj["ms_per_step"] * 1e3
    lines += [
        "",
        f"Dominant kernel `{a.title}`: **{kernel_us:.1f} µs** per timed step "
        f"({flops / kernel_us / 1e6:.1f} TFLOP/s, {100 * flops / kernel_us / 1e6 / peak:.1f}% of {peak}). "
        f"`bench.py` in the same profiled run (HIP events on the launch stream over the {steps} steps): "
        f"**{step_us:.1f} µs** per step, primitive `{cfg['primitive']}`. Algorithmic bytes over the kernel time: "
        f"{alg / kernel_us / 1e3:.1f} GB/s ({100 * alg / kernel_us / 1e3 / 8000:.1f}% of 8 TB/s).",
        "",
        "## HBM traffic and counters per dispatch (PMC)", "",
        "| FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes (scaled) | Algorithmic bytes | Ratio | MFMA busy | MFMA busy, floor | LDS bank conflicts / LDS active |",
        "|---:|---:|---:|---:|---:|---:|---:|---:|",
        f"| {fetch:.1f} | {write:.1f} | {traffic:.4g} | {alg:.4g} | {traffic / alg:.2f} | {100 * busy:.1f}% | "
        f"{100 * busy_floor:.1f}% | {conflict:.3f} |",
        "",
        f"Scales from the copy calibration (a 256 MiB device copy reads {cf:.1f} KiB and writes {cw:.1f} KiB "
        f"per dispatch): FETCH_SIZE × {fs:.4f}, WRITE_SIZE × {ws:.4f}.",
        "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs × GRBM_GUI_ACTIVE / 8 XCDs).",
        f"MFMA busy, floor = SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs / (the traced kernel time × "
        f"{PEAK_CLOCK_HZ / 1e9:.1f} GHz, the highest shader clock): the busy fraction is at least this at any clock. "
        "GRBM_GUI_ACTIVE spans the counter window, which adds several µs to each dispatch, so the first ratio "
        "understates kernels of a few tens of µs.",
    ]
    with open(a.out, "w") as f:
        f.write("\n".join(lines) + "\n")
    tj_path = os.path.join(REPO, "profiles", "traffic.json")
    tj = json.load(open(tj_path)) if os.path.exists(tj_path) else {}
    tj[a.workload] = {"kernel": a.title, "hbm_bytes_per_launch": int(traffic), "algorithmic_bytes": int(alg),
                      "kernel_us_timed_mean": round(kernel_us, 2), "mfma_busy": round(busy, 4),
                      "mfma_busy_floor": round(busy_floor, 4),
                      "profile": os.path.relpath(os.path.abspath(a.out), REPO)}
    with open(tj_path, "w") as f:
        json.dump(tj, f, indent=1)


if __name__ == "__main__":
    main()
