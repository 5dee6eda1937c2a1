#!/usr/bin/env python3
"""MFMA busy over the cycles the CUs run a kernel's waves, per profiled workload.

One rocprofv3 pass per workload, under --dir/<workload>/:
  rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE --output-format csv \\
      -d <dir>/<workload> -o run -- python3 bench.py --no-cpu --no-overhead --no-configs <args> \\
      --steps 3 --warmup 1 --warm-ms 0

SQ_VALU_MFMA_BUSY_CYCLES is summed over the SIMDs (4 per CU) and SQ_BUSY_CU_CYCLES over the CUs, so
MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (4 x SQ_BUSY_CU_CYCLES) counts only cycles in which a CU holds
the kernel's waves.  The counter's description gives SQ_BUSY_CU_CYCLES in quad-cycles; on MI355X its
sum reads as cycles: the fp32 kernels that run at 0.98 of the MFMA peak read 98.6-99.7% this way and
would read a quarter of that with a quad-cycle reading, which their FLOP rate rules out.  The GRBM_GUI_ACTIVE ratio beside it spans the whole counter window, which adds
several microseconds per dispatch and understates kernels of a few tens of microseconds.

  python3 flash-train_amd/bench/mfma_busy_summary.py --dir gpurun_out/busy \\
      --case square_8192 fp32_gemm_dma "" ... --out profiles/mfma_busy_cu_active.md
"""

from __future__ import annotations

import argparse
import collections
import csv
import os


def counters(path: str, match: str) -> dict:
    agg = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            if match in r["Kernel_Name"]:
                agg[r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: (sum(v) / len(v), len(v)) for k, v in agg.items()}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--dir", required=True)
    ap.add_argument("--case", nargs=3, action="append", required=True, metavar=("WORKLOAD", "KERNEL", "ARGS"),
                    help="workload (subfolder of --dir), substring of its dominant kernel, bench.py arguments")
    ap.add_argument("--out", required=True)
    a = ap.parse_args()
    lines = [
        "# MFMA busy over CU-active cycles, per profiled workload", "",
        "Commands, run from the repository root on the MI355X box after "
        "`cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT`, one per workload, then the summary:", "", "```",
    ]
    for wl, _, args in a.case:
        lines.append(f"rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE --output-format csv "
                     f"-d {a.dir}/{wl} -o run -- python3 bench.py --no-cpu --no-overhead --no-configs {args} "
                     "--steps 3 --warmup 1 --warm-ms 0".replace("  ", " "))
    cases = " ".join(f"--case {wl} {k} \"{args}\"" for wl, k, args in a.case)
    lines += [f"python3 flash-train_amd/bench/mfma_busy_summary.py --dir {a.dir} {cases} --out {a.out}", "```", "",
              "| Workload | Kernel | Dispatches | MFMA busy, CU-active | MFMA busy, GRBM_GUI_ACTIVE window |",
              "|---|---|---:|---:|---:|"]
    for wl, kern, _ in a.case:
        c = counters(os.path.join(a.dir, wl, "run_counter_collection.csv"), kern)
        mf, n = c["SQ_VALU_MFMA_BUSY_CYCLES"]
        cu = c["SQ_BUSY_CU_CYCLES"][0]
        gr = c["GRBM_GUI_ACTIVE"][0]
        lines.append(f"| `{wl}` | `{kern}` | {n} | {100 * mf / (4 * cu):.1f}% | {100 * mf / (1024 * gr / 8):.1f}% |")
    lines += ["", "MFMA busy, CU-active = SQ_VALU_MFMA_BUSY_CYCLES / (4 SIMDs per CU × SQ_BUSY_CU_CYCLES). "
              "The window column is SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs × GRBM_GUI_ACTIVE / 8 XCDs), the "
              "ratio the per-kernel pages report. SQ_BUSY_CU_CYCLES is read as cycles (its description says "
              "quad-cycles): the fp32 kernels that run at 0.98 of the MFMA peak then read 98.6–99.7%, and a "
              "quad-cycle reading would put them at a quarter of that, which their FLOP rate rules out. On "
              "short kernels the window column falls and the CU-active one does not."]
    with open(a.out, "w") as f:
        f.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
