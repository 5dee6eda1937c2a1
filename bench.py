#!/usr/bin/env python3
"""FP32 GEMM throughput of the flash-train MI355X path (one GPU).

A step is one execution of a cached Plan (ftrainPlanExecutePrimitive, primitive
0) on the headline BASELINE workload, m = n = k = 8192, a, b ~ U(-1, 1) from a
CPU torch.Generator seeded 2026, alpha 1, beta 0, no c; inputs are resident in
HBM before timing.  Prints ONE JSON line (rank 0) with the metric, the
roofline of the dominant kernel, the cached-Plan host overhead, and a CPU
baseline.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.join(REPO, "flash-train_amd")
for _p in (PKG_ROOT, REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

FP32_MATRIX_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix (AMD spec)
HALF_MATRIX_PEAK_TFLOPS = 2500.0  # MI355X dense BF16 / FP16 matrix (AMD spec, no sparsity)
HBM_PEAK_GBS = 8000.0
METRIC = "FP32 GEMM TFLOP/s and % of MFMA FP32 peak at 8192³; µs/call on cached Plan"


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


def plan_overhead() -> dict | None:
    """Runs the C++ probe (separate process) on BASELINE config 5e (127, 97, 33)."""
    exe = os.path.join(PKG_ROOT, "bench", "plan_overhead")
    if not os.path.exists(exe):
        return None
    try:
        out = subprocess.run([exe, "127", "97", "33", "10000"], capture_output=True, text=True, timeout=120)
        return json.loads(out.stdout.strip().splitlines()[-1]) if out.returncode == 0 else {"error": out.stderr[-400:]}
    except Exception as e:  # report, do not fail the bench
        return {"error": str(e)}


def torch_binding_overhead(iters: int = 2000) -> dict:
    """Host microseconds per flash_train.torch.gemm call on BASELINE config 5e (127, 97, 33)."""
    import torch

    import flash_train.torch as ftt

    g = torch.Generator().manual_seed(2026)
    a = torch.randn(127, 33, generator=g).cuda()
    b = torch.randn(33, 97, generator=g).cuda()
    for _ in range(50):
        ftt.gemm(a, b)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        ftt.gemm(a, b)
    host = (time.perf_counter() - t0) / iters * 1e6
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(iters):
        torch.matmul(a, b)
    ref = (time.perf_counter() - t1) / iters * 1e6
    torch.cuda.synchronize()
    return {"flash_train_torch_gemm_host_us": round(host, 2), "torch_matmul_host_us": round(ref, 2), "iters": iters}


def traffic_from_profiles(workload: str) -> float | None:
    """HBM bytes per launch of the workload's kernel: the committed rocprofv3 PMC figure
    (FETCH_SIZE + WRITE_SIZE, each scaled by the copy-kernel calibration), if one exists."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(workload, {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(a, b, alpha: float, beta: float, budget_s: float) -> dict:
    """The oracle's restatement of the reference kernel (fp32, in-order k sum), on a row sample."""
    from oracle import oracle

    import numpy as np

    k = a.shape[1]
    n = b.shape[1]
    a_np, b_np = a.numpy(), b.numpy()
    # Two probes: the first (4 rows) also pays thread start-up, so it sizes a
    # second ~1 s probe whose rate then sizes the sample to budget_s.
    rows = 4
    for target_s in (1.0, budget_s):
        t0 = time.perf_counter()
        oracle.gemm_ref(a_np[:rows], b_np, None, alpha, beta)
        dt = max(time.perf_counter() - t0, 1e-6)
        rows = int(min(a.shape[0], max(rows, rows * target_s / dt)))
    t0 = time.perf_counter()
    oracle.gemm_ref(a_np[:rows], b_np, None, alpha, beta)
    dt = time.perf_counter() - t0
    tflops = 2.0 * rows * n * k / dt / 1e12
    return {"value": round(tflops, 5), "unit": "TFLOP/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{rows} of {a.shape[0]} rows of the workload ({rows}x{n}x{k}), {dt:.1f} s, "
                      f"oracle/gemm_oracle.c ft_oracle_gemm_ref with OpenMP"}


def torch_cpu_matmul(a, b, budget_s: float) -> dict:
    import torch

    torch.set_num_threads(os.cpu_count() or 1)
    rows = 256
    t0 = time.perf_counter()
    torch.matmul(a[:rows], b)
    dt = max(time.perf_counter() - t0, 1e-6)
    rows = int(min(a.shape[0], max(rows, rows * budget_s / dt)))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        torch.matmul(a[:rows], b)
        times.append(time.perf_counter() - t0)
    dt = sorted(times)[1]
    return {"value": round(2.0 * rows * b.shape[1] * a.shape[1] / dt / 1e12, 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "sample": f"{rows}x{b.shape[1]}x{a.shape[1]}, median of 3"}


def expert_rows(m: int, experts: int) -> list:
    """Uneven token counts per expert (deterministic), summing to m; none a multiple of the tile."""
    w = [1.0 + 0.6 * math.sin(1.7 * e + 0.3) for e in range(experts)]
    rows = [int(m * x / sum(w)) for x in w]
    rows[-1] += m - sum(rows)
    return rows


def grouped_core(workload: str, E: int, dtype: str, steps: int, warmup: int, warm_ms: float = 25.0) -> dict:
    """One GroupedABCDGemm Plan (Primitive 0) over E experts: the workload's m rows split unevenly, each
    expert with its own k x n weight.  Timed with HIP events on the launch stream; 8 sampled rows of every
    expert checked against fp64."""
    import numpy as np
    import torch

    import flash_train.capi as capi
    from oracle import oracle

    a_h, b_h, c_h, cfg = oracle.seeded_inputs(workload)
    m, n, k = cfg["m"], cfg["n"], cfg["k"]
    rows = expert_rows(m, E)
    dt = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}[dtype]
    # Expert e's weight: the workload's b with its columns rotated by 97·e (distinct memory, same distribution).
    b_all = torch.stack([torch.roll(b_h, 97 * e, dims=1) for e in range(E)]).to(dt)
    a_h = a_h.to(dt)
    a, b = a_h.cuda(), b_all.cuda()
    c = c_h.cuda() if c_h is not None else None
    d = torch.empty(m, n, device="cuda")
    ops = capi.GroupedOps("abcd")
    al, be = capi.HostScalar(cfg["alpha"]), capi.HostScalar(cfg["beta"])
    dims_mn = [(r, n) for r in rows]
    cspec = capi.GroupedSpec(capi.matrix(c) if c is not None else capi.View(None, [m, n]), E, dims=dims_mn)
    gargs = ops.args(a=capi.GroupedSpec(capi.matrix(a), E, dims=[(r, k) for r in rows]),
                     b=capi.GroupedSpec(capi.matrix(b[0]), E), c=cspec,
                     d=capi.GroupedSpec(capi.matrix(d), E, dims=dims_mn), alpha=al.view, beta=be.view)
    plan = gargs.plan()
    gargs.close()
    name = plan.name(0)
    log(f"grouped {workload} ({m}x{n}x{k}) over {E} experts, rows {rows}; primitive 0 = {name}")
    stream = torch.cuda.Stream()
    h = stream.cuda_stream
    with torch.cuda.stream(stream):
        warm_up(lambda: plan.execute(0, h), stream, warmup, warm_ms)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            plan.execute(0, h)
        stop.record(stream)
        torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps

    rng = np.random.default_rng(1)
    ok, worst, row0 = True, 0.0, 0
    for e, r in enumerate(rows):
        pick = np.sort(rng.choice(r, size=min(8, r), replace=False)) + row0
        ref = oracle.sampled_rows_f64(a_h.float(), b_all[e].float(), c_h, cfg["alpha"], cfg["beta"], pick)
        rep = oracle.tolerance_check(d[torch.as_tensor(pick).cuda()].cpu().numpy(), ref, k)
        ok, worst = ok and rep["ok"], max(worst, rep["max_abs_err"] / max(rep["bound"], 1e-30))
        row0 += r
    del a, b, c, d, plan
    torch.cuda.empty_cache()

    half = dtype != "fp32"
    flops = 2.0 * m * n * k
    tflops = flops / (ms * 1e-3) / 1e12
    peak = HALF_MATRIX_PEAK_TFLOPS if half else FP32_MATRIX_PEAK_TFLOPS
    eb = 2.0 if half else 4.0
    alg_bytes = eb * (m * k + E * k * n) + 4.0 * m * n * (2 if c_h is not None else 1)
    key = f"grouped_{workload}_e{E}"
    return {"workload": key + ("" if not half else f"_{dtype}"), "m": m, "n": n, "k": k, "experts": E,
            "rows": rows, "dtype": dtype, "c": c_h is not None, "primitive": name, "steps": steps,
            "ms": round(ms, 5), "tflops": round(tflops, 3),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": peak, "unit": "TFLOP/s",
                         "frac": round(tflops / peak, 4),
                         "traffic": traffic_from_profiles(key + ("" if not half else f"_{dtype}_nn")),
                         "algorithmic_bytes": alg_bytes, "algorithmic_flops": flops},
            "parity": {"rows_checked": int(sum(min(8, r) for r in rows)), "worst_err_over_bound": worst,
                       "ok": bool(ok)}}


def grouped_wgrad_core(E: int, dtype: str, steps: int, warmup: int, tokens_total: int = 16384, m: int = 4096,
                       n: int = 14336) -> dict:
    """Mixture-of-experts weight gradient, one GroupedABGemm Plan (Primitive 0): dW_e = X_e^T @ dY_e over
    each expert's tokens (the reduction depth, uneven and not a multiple of any tile: expert_rows), X the
    packed m-wide activations, dY the packed n-wide output gradients, fp32 dW.  Timed with HIP events on
    the launch stream; 4 sampled rows of every expert's dW checked against fp64."""
    import numpy as np
    import torch

    import flash_train.capi as capi
    from oracle import oracle

    tokens = expert_rows(tokens_total, E)
    dt = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}[dtype]
    g = torch.Generator().manual_seed(2026)
    X_h = torch.randn(tokens_total, m, generator=g).to(dt)
    dY_h = torch.randn(tokens_total, n, generator=g).to(dt)
    X, dY = X_h.cuda(), dY_h.cuda()
    d_all = torch.empty(E, m, n, device="cuda")
    offs = [sum(tokens[:e]) for e in range(E)]
    ops = capi.GroupedOps("ab")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    gargs = ops.args(
        a=capi.GroupedSpec(capi.matrix(X), E, dims=[(m, t) for t in tokens], strides=[(1, m)] * E,
                           offsets=[o * m for o in offs]),
        b=capi.GroupedSpec(capi.matrix(dY), E, dims=[(t, n) for t in tokens]),
        c=[capi.View(None, [m, n], numeric_type=capi.TORCH_NUMERIC_TYPES[torch.float32]) for _ in range(E)],
        d=[capi.matrix(d_all[e]) for e in range(E)], alpha=al.view, beta=be.view)
    plan = gargs.plan()
    gargs.close()
    name = plan.name(0)
    log(f"grouped weight gradient {m}x{n} over {E} experts, tokens {tokens}; primitive 0 = {name}")
    stream = torch.cuda.Stream()
    h = stream.cuda_stream
    with torch.cuda.stream(stream):
        warm_up(lambda: plan.execute(0, h), stream, warmup, 25.0)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            plan.execute(0, h)
        stop.record(stream)
        torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps

    rng = np.random.default_rng(3)
    ok, worst = True, 0.0
    for e, t in enumerate(tokens):
        rows = np.sort(rng.choice(m, size=4, replace=False))
        o = offs[e]
        ref = (X_h[o:o + t, rows].double().t() @ dY_h[o:o + t].double()).numpy()
        rep = oracle.tolerance_check(d_all[e][torch.as_tensor(rows).cuda()].cpu().numpy(), ref, max(t, 1))
        ok, worst = ok and rep["ok"], max(worst, rep["max_abs_err"] / max(rep["bound"], 1e-30))
    del X, dY, d_all, plan
    torch.cuda.empty_cache()

    half = dtype != "fp32"
    flops = 2.0 * tokens_total * m * n
    tflops = flops / (ms * 1e-3) / 1e12
    peak = HALF_MATRIX_PEAK_TFLOPS if half else FP32_MATRIX_PEAK_TFLOPS
    eb = 2.0 if half else 4.0
    alg_bytes = eb * tokens_total * (m + n) + 4.0 * E * m * n
    return {"workload": f"grouped_wgrad_e{E}" + ("" if not half else f"_{dtype}"), "m": m, "n": n,
            "k": tokens_total, "experts": E, "tokens": tokens, "dtype": dtype, "primitive": name, "steps": steps,
            "ms": round(ms, 5), "tflops": round(tflops, 3),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": peak, "unit": "TFLOP/s",
                         "frac": round(tflops / peak, 4), "traffic": None,
                         "algorithmic_bytes": alg_bytes, "algorithmic_flops": flops},
            "parity": {"rows_checked": 4 * E, "worst_err_over_bound": worst, "ok": bool(ok)}}


def run_grouped(args) -> None:
    """--grouped E: one step = one GroupedABCDGemm launch sequence over all experts; prints one JSON line."""
    g = grouped_core(args.workload, args.grouped, args.dtype, args.steps, args.warmup, args.warm_ms)
    print(json.dumps({
        "metric": METRIC, "value": g["tflops"], "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(g["ms"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": args.dtype,
        "data": "synthetic (seeded CPU torch.Generator 2026; expert weights are column rotations of b)",
        "config": {"workload": g["workload"], "m": g["m"], "n": g["n"], "k": g["k"], "experts": g["experts"],
                   "rows": g["rows"], "c": g["c"], "primitive": g["primitive"], "parallelism": "single GPU"},
        "pct_of_matrix_peak": round(100.0 * g["roofline"]["frac"], 2),
        "roofline": dict(g["roofline"], kernel_ms=round(g["ms"], 4), kernel=g["primitive"]),
        "parity": g["parity"],
    }), flush=True)


# BASELINE configurations timed after the headline (BASELINE.json configs[0..4]):
# name -> steps on one cached Plan (configs[3] asks for 100 iterations per MLP shape).
CONFIG_STEPS = {
    "readme_128x96x64": 200,
    "square_4096_beta": 50,
    "mlp_fwd": 100,
    "mlp_dgrad": 100,
    "skinny_64x4096x4096": 200,
    "skinny_4096x64x4096": 200,
    "splitk_256x256x65536": 200,
    "gemv_1x8192x8192": 200,
    "odd_127x97x33": 200,
}


def warm_up(call, stream, calls: int, min_ms: float = 25.0) -> None:
    """`calls` untimed calls, then more until about `min_ms` of GPU work has run: a few calls of a
    short kernel leave the clock below its steady-state value (measured on MI355X: 256x256x65536
    73 us right after 10 warm-up calls, 66 us once warm)."""
    import torch

    for _ in range(calls):
        call()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for _ in range(10):
        call()
    e.record(stream)
    torch.cuda.synchronize()
    per = max(s.elapsed_time(e) / 10, 1e-3)
    for _ in range(min(int(min_ms / per), 20000)):
        call()
    torch.cuda.synchronize()


def time_steps(plan, index: int, stream, steps: int, warmup: int, block: int = 10, workspace=(0, 0)) -> dict:
    """HIP events on the launch stream around blocks of `block` back-to-back calls: the mean over
    all steps and the median of the block means (ms per call).  An event between every two calls
    adds a marker to the queue that costs about 2-3 us next to a 25 us kernel; the per-call event
    median is reported beside it."""
    import torch

    h = stream.cuda_stream
    blocks = max(1, steps // block)
    with torch.cuda.stream(stream):
        warm_up(lambda: plan.execute(index, h, *workspace), stream, warmup)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(blocks + 1)]
        ev[0].record(stream)
        for i in range(blocks):
            for _ in range(block):
                plan.execute(index, h, *workspace)
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        per_block = sorted(ev[i].elapsed_time(ev[i + 1]) / block for i in range(blocks))
        one = [torch.cuda.Event(enable_timing=True) for _ in range(block + 1)]
        one[0].record(stream)
        for i in range(block):
            plan.execute(index, h, *workspace)
            one[i + 1].record(stream)
        torch.cuda.synchronize()
    per_call = sorted(one[i].elapsed_time(one[i + 1]) for i in range(block))
    return {"mean_ms": ev[0].elapsed_time(ev[-1]) / (blocks * block), "median_ms": per_block[blocks // 2],
            "event_per_call_median_ms": per_call[block // 2]}


def parity_rows(oracle, a_h, b_h, c_h, cfg, d, rows_wanted: int = 64, ref=None) -> tuple:
    """fp64 check of sampled rows (all rows when m is small) against the north-star bar, and how far
    inside it the result is (a subtle pipeline slip would show as a ratio far above the usual 1e-3).
    Returns the report and the (rows, fp64 reference) pair, which later checks of the same inputs reuse."""
    import numpy as np
    import torch

    m = cfg["m"]
    if ref is None:
        rows = np.arange(m) if m <= rows_wanted else np.sort(
            np.random.default_rng(1).choice(m, size=rows_wanted, replace=False))
        ref = (rows, oracle.sampled_rows_f64(a_h.float(), b_h.float(), c_h, cfg["alpha"], cfg["beta"], rows))
    rows, want = ref
    rep = oracle.tolerance_check(d[torch.as_tensor(rows).cuda()].cpu().numpy(), want, cfg["k"])
    ratio = rep["max_abs_err"] / rep["bound"] if rep["bound"] > 0 else 0.0
    return ({"rows_checked": int(len(rows)), "max_abs_err": rep["max_abs_err"], "bound": rep["bound"],
             "err_over_bound": ratio, "ok": bool(rep["ok"] and ratio <= 1e-2)}, ref)


# BASELINE configs whose every Primitive is timed as well (the reference harness's L4 tier,
# benchmarks/csrc/ftrain_bench.cpp:158-166): config 5 ("verifies Finder choice") and 4096³ + c.
PRIMITIVE_MATRIX = ("square_4096_beta", "skinny_64x4096x4096", "skinny_4096x64x4096", "splitk_256x256x65536",
                    "gemv_1x8192x8192", "odd_127x97x33")


def primitive_matrix(plan, stream, d, check, steps: int, passes: int = 2) -> dict:
    """Every Primitive of the Plan, timed like Primitive 0 (blocks of 10 back-to-back calls) with one
    caller workspace as large as the largest requirement, each result checked.  The matrix is walked
    `passes` times and each Primitive keeps its best median, so a clock still ramping after a pause
    (the parity check runs on the host) does not count against whichever Primitive comes first.
    `pick_loss` is how much slower the Finder's pick (Primitive 0) runs than the fastest Primitive."""
    import torch

    names = plan.names()
    need = max(plan.workspace_bytes(i) for i in range(len(names)))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    best_ms = [math.inf] * len(names)
    ok = [True] * len(names)
    for p in range(passes):
        for i in range(len(names)):
            d.fill_(float("nan"))
            # First pass 20 steps; later ones up to `steps`, about 60 ms of calls at most (the
            # Primitive's first-pass time), so slow Primitives do not stretch the run.
            n = min(steps, 20) if p == 0 else min(steps, max(20, int(60.0 / max(best_ms[i], 1e-3)) // 10 * 10))
            t = time_steps(plan, i, stream, n, warmup=3, workspace=(ws.data_ptr(), ws.numel()))
            best_ms[i] = min(best_ms[i], t["median_ms"])
            ok[i] = ok[i] and bool(check()["ok"])
    rows = [{"index": i, "primitive": nm, "workspace_bytes": plan.workspace_bytes(i),
             "median_ms": round(best_ms[i], 5), "ok": ok[i]} for i, nm in enumerate(names)]
    best = min(rows, key=lambda r: r["median_ms"])
    del ws
    return {"primitives": rows, "fastest": best["primitive"],
            "pick_loss": round(rows[0]["median_ms"] / best["median_ms"] - 1.0, 4)}


def run_config(name: str, steps: int, dtype: str = "fp32", all_primitives: bool = False) -> dict:
    """One BASELINE config on one cached Plan (Primitive 0): median step time, rate, roofline, parity;
    with `all_primitives`, the per-Primitive matrix too."""
    import torch

    import flash_train.capi as capi
    from oracle import oracle

    a_h, b_h, c_h, cfg = oracle.seeded_inputs(name)
    half = dtype != "fp32"
    if half:
        dt = torch.bfloat16 if dtype == "bf16" else torch.float16
        a_h, b_h = a_h.to(dt), b_h.to(dt)
    m, n, k = cfg["m"], cfg["n"], cfg["k"]
    a, b = a_h.cuda(), b_h.cuda()
    c = c_h.cuda() if c_h is not None else None
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, c, d, cfg["alpha"], cfg["beta"])
    stream = torch.cuda.Stream()
    t = time_steps(plan, 0, stream, steps, warmup=max(3, steps // 20))
    ms = t["median_ms"]
    parity, ref = parity_rows(oracle, a_h, b_h, c_h, cfg, d)
    flops = 2.0 * m * n * k
    eb = 2.0 if half else 4.0
    alg_bytes = eb * (m * k + k * n) + 4.0 * m * n * (2 if c is not None else 1)
    peak = HALF_MATRIX_PEAK_TFLOPS if half else FP32_MATRIX_PEAK_TFLOPS
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    hbm_bound = flops / alg_bytes < peak * 1e12 / (HBM_PEAK_GBS * 1e9)
    key = name if not half else f"{name}_{dtype}"
    out = {"workload": key, "m": m, "n": n, "k": k, "dtype": dtype, "c": c is not None,
           "primitive": plan.name(0), "steps": steps, "median_ms": round(ms, 5), "mean_ms": round(t["mean_ms"], 5),
           "event_per_call_median_ms": round(t["event_per_call_median_ms"], 5),
           "tflops": round(tflops, 3), "gbs": round(gbs, 1),
           "roofline": {"bound": "hbm" if hbm_bound else "mfma",
                        "frac": round(gbs / HBM_PEAK_GBS if hbm_bound else tflops / peak, 4),
                        "peak": HBM_PEAK_GBS if hbm_bound else peak, "unit": "GB/s" if hbm_bound else "TFLOP/s",
                        "traffic": traffic_from_profiles(name if not half else f"{name}_{dtype}_nn")},
           "parity": parity}
    if all_primitives:
        # Up to as many steps as Primitive 0's own timing: with only two blocks of 10, the median is
        # the first block, which a kernel shorter than the host's launch path spends waiting for the
        # queue to fill (bf16 64x4096x4096: 18.6 against 12.6 us).
        out.update(primitive_matrix(plan, stream, d, lambda: parity_rows(oracle, a_h, b_h, c_h, cfg, d, ref=ref)[0],
                                    steps=max(20, steps)))
    del a, b, c, d, plan
    torch.cuda.empty_cache()
    return out


# The reference's own benchmark shapes, (m, k, n): its published table (docs/benchmarks/gemm-fp32.md:10-42)
# and its "standard" suite (benchmarks/ftrain_bench/ops/gemm.py:41-52).
REFERENCE_SHAPES = ((64, 64, 64), (128, 128, 128), (256, 256, 256), (512, 512, 512), (1024, 1024, 1024),
                    (2048, 2048, 2048), (4096, 4096, 4096), (8192, 8192, 8192), (1024, 4096, 4096),
                    (4096, 1024, 11008))


def reference_measure(fn, warmup: int = 10, target_ms: float = 200.0, lo: int = 10, hi: int = 200) -> float:
    """The reference harness's timing policy (benchmarks/ftrain_bench/timing.py:21-43): warm-up, then
    each call bracketed by events on the current stream and synchronised, the iteration count adapted to
    about 200 ms within [10, 200]; the median in ms."""
    import statistics

    import torch

    def once():
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e)

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    iters = max(lo, min(hi, int(target_ms / max(once(), 1e-3)) + 1))
    return statistics.median(once() for _ in range(iters))


def reference_suite() -> list:
    """L1 (flash_train.torch.gemm), L2 (ftrainGemm, through ctypes), L3 (cached Plan, Primitive 0; the
    reference's L4 for Primitive 0 is the same call) and the torch.matmul baseline per reference shape,
    with a, b ~ N(0, 1) drawn as the reference harness draws them (seed 2026)."""
    import torch

    import flash_train.capi as capi
    import flash_train.torch as ftt

    out = []
    for m, k, n in REFERENCE_SHAPES:
        torch.manual_seed(2026)
        a = torch.randn((m, k), device="cuda")
        b = torch.randn((k, n), device="cuda")
        d = torch.empty(m, n, device="cuda")
        plan = capi.plan_for(a, b, None, d, 1.0, 0.0)
        h = torch.cuda.current_stream().cuda_stream
        l3 = reference_measure(lambda: plan.execute(0, h))
        al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
        va, vb, vc, vd = capi.matrix(a), capi.matrix(b), capi.View(None, [m, n]), capi.matrix(d)
        l2_call = lambda: capi.gemm_status(va, vb, vc, vd, al.view, be.view, stream=h)
        if l2_call() != capi.SUCCESS:
            raise RuntimeError(f"ftrainGemm {m}x{k}x{n}: {capi.last_message()}")
        l2 = reference_measure(l2_call)
        l1 = reference_measure(lambda: ftt.gemm(a, b))
        base = reference_measure(lambda: torch.matmul(a, b))
        flops = 2.0 * m * n * k
        out.append({"shape_mkn": [m, k, n], "primitive": plan.name(0), "l3_plan_ms": round(l3, 5),
                    "l2_ftrain_gemm_ms": round(l2, 5), "l1_torch_gemm_ms": round(l1, 5),
                    "torch_matmul_ms": round(base, 5),
                    "l3_tflops": round(flops / (l3 * 1e-3) / 1e12, 3)})
        del a, b, d, plan
    torch.cuda.empty_cache()
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="square_8192")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work")
    ap.add_argument("--layout", default="nn", choices=("nn", "tn", "nt", "tt"),
                    help="operand orientation: t = a (first letter) or b (second) stored column-major, "
                         "passed with explicit strides")
    ap.add_argument("--dtype", default="fp32", choices=("fp32", "bf16", "fp16"),
                    help="element type of a and b (c and d stay fp32; accumulation is fp32)")
    ap.add_argument("--warm-ms", type=float, default=25.0,
                    help="GPU milliseconds of extra warm-up before timing a workload other than the fp32 headline "
                         "(0 for counter-collection runs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--no-overhead", action="store_true", help="skip the cached-Plan host-overhead probe")
    ap.add_argument("--grouped", type=int, default=0, metavar="E",
                    help="grouped GEMM (GroupedABCDGemm): the workload's m rows split unevenly over E experts, "
                         "each with its own k x n weight (mixture-of-experts forward)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other BASELINE configs (the `configs` key of the JSON line)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 5 device copies of 256 MiB (the known-size kernel that scales the PMC "
                         "FETCH_SIZE / WRITE_SIZE counters into bytes)")
    args = ap.parse_args()

    if args.copy_calibration:
        import torch

        x = torch.empty(64 * 1024 * 1024, device="cuda")
        y = torch.empty_like(x)
        for _ in range(5):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": x.numel() * 4, "bytes_written": y.numel() * 4}))
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the GEMM path on a single MI355X "
              "and has no multi-GPU sharding; use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    import flash_train.capi as capi
    from oracle import oracle

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    a_h, b_h, c_h, cfg = oracle.seeded_inputs(args.workload)
    if args.grouped:
        run_grouped(args)
        return
    m, n, k = cfg["m"], cfg["n"], cfg["k"]
    half = args.dtype != "fp32"
    if half:
        # The 16-bit inputs are the fp32 draws rounded; the parity reference uses the rounded values.
        dt = torch.bfloat16 if args.dtype == "bf16" else torch.float16
        a_h, b_h = a_h.to(dt), b_h.to(dt)
    # Column-major operands: the transpose is stored contiguously and viewed back.
    a = a_h.t().contiguous().cuda().t() if args.layout[0] == "t" else a_h.cuda()
    b = b_h.t().contiguous().cuda().t() if args.layout[1] == "t" else b_h.cuda()
    c = c_h.cuda() if c_h is not None else None
    d = torch.empty(m, n, device="cuda")
    stream = torch.cuda.Stream()
    plan = capi.plan_for(a, b, c, d, cfg["alpha"], cfg["beta"])
    name = plan.name(0)
    log(f"workload {args.workload} ({m}x{n}x{k}); primitive 0 = {name}; plan = {plan.names()}")

    h = stream.cuda_stream
    with torch.cuda.stream(stream):
        # The headline's W warm-up steps (7 ms each) reach steady state; the other workloads' short
        # steps get a time-based warm-up on top.
        headline = args.workload == "square_8192" and args.dtype == "fp32" and args.layout == "nn"
        warm_up(lambda: plan.execute(0, h), stream, args.warmup, 0.0 if headline else args.warm_ms)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(stream)
        for _ in range(args.steps):
            plan.execute(0, h)
        stop.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms = start.elapsed_time(stop) / args.steps

    # Parity spot check of the benchmarked output (64 sampled rows, fp64).
    import numpy as np

    rows = np.sort(np.random.default_rng(1).choice(m, size=min(64, m), replace=False))
    ref = oracle.sampled_rows_f64(a_h.float(), b_h.float(), c_h, cfg["alpha"], cfg["beta"], rows)
    rep = oracle.tolerance_check(d[torch.as_tensor(rows).cuda()].cpu().numpy(), ref, k)

    flops = 2.0 * m * n * k
    tflops = flops / (ms * 1e-3) / 1e12
    in_bytes = 2.0 if half else 4.0
    alg_bytes = in_bytes * (m * k + k * n) + 4.0 * m * n * (2 if c is not None else 1)
    peak_tflops = HALF_MATRIX_PEAK_TFLOPS if half else FP32_MATRIX_PEAK_TFLOPS
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    # Roofline bound: arithmetic intensity against the ridge point (157.3 TFLOP/s / 8 TB/s).
    hbm_bound = flops / alg_bytes < peak_tflops * 1e12 / (HBM_PEAK_GBS * 1e9)
    if hbm_bound:
        roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(gbs / HBM_PEAK_GBS, 4)}
    else:
        roofline = {"bound": "mfma", "achieved": round(tflops, 3), "peak": peak_tflops,
                    "unit": "TFLOP/s", "frac": round(tflops / peak_tflops, 4)}
    traffic_key = args.workload + ("" if args.dtype == "fp32" and args.layout == "nn" else f"_{args.dtype}_{args.layout}")
    roofline.update({"traffic": traffic_from_profiles(traffic_key), "algorithmic_bytes": alg_bytes,
                     "algorithmic_flops": flops, "kernel_ms": round(ms, 4), "kernel": name})
    overhead = None if args.no_overhead else plan_overhead()
    if overhead is not None and "error" not in overhead:
        overhead["torch_binding"] = torch_binding_overhead()

    result = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded CPU torch.Generator 2026; BASELINE.json distributions)",
        "config": {"workload": args.workload, "layout": args.layout, "m": m, "n": n, "k": k,
                   "alpha": cfg["alpha"], "beta": cfg["beta"],
                   "c": c is not None, "primitive": name, "parallelism": "single GPU"},
        "pct_of_matrix_peak": round(100.0 * tflops / peak_tflops, 2),
        "roofline": roofline,
        "plan_overhead": overhead,
        "parity": {"rows_checked": int(len(rows)), "max_abs_err": rep["max_abs_err"], "bound": rep["bound"],
                   "err_over_bound": rep["max_abs_err"] / rep["bound"] if rep["bound"] > 0 else 0.0,
                   "ok": bool(rep["ok"] and rep["max_abs_err"] <= 1e-2 * rep["bound"])},
        "wall_s_timed": round(wall, 3),
    }
    if not args.no_configs and not half and args.layout == "nn" and args.workload == "square_8192":
        del a, b, c, d, plan
        torch.cuda.empty_cache()
        configs = []
        for name, steps in CONFIG_STEPS.items():
            log(f"config {name}")
            configs.append(run_config(name, steps, all_primitives=name in PRIMITIVE_MATRIX))
        # Grouped GEMM (mixture-of-experts forward) and bf16 inputs on the BASELINE shapes.
        for name, steps in (("square_8192", 50), ("mlp_fwd", 50), ("skinny_64x4096x4096", 200)):
            log(f"config {name} bf16")
            configs.append(run_config(name, steps, dtype="bf16", all_primitives=True))
        for experts in (8, 64):
            log(f"config grouped mlp_fwd over {experts} experts")
            configs.append(grouped_core("mlp_fwd", experts, "fp32", steps=10, warmup=2))
        for experts in (8, 64):
            log(f"config grouped mlp_fwd over {experts} experts bf16")
            configs.append(grouped_core("mlp_fwd", experts, "bf16", steps=20, warmup=2))
        for dtype, steps in (("fp32", 10), ("bf16", 20)):
            log(f"config grouped weight gradient over 8 experts {dtype}")
            configs.append(grouped_wgrad_core(8, dtype, steps=steps, warmup=2))
        result["configs"] = configs
        log("reference benchmark shapes")
        result["reference_suite"] = reference_suite()
    if not args.no_cpu and not half:
        result["cpu_baseline"] = cpu_baseline(a_h, b_h, cfg["alpha"], cfg["beta"], args.cpu_budget)
        result["cpu_torch_matmul"] = torch_cpu_matmul(a_h, b_h, min(args.cpu_budget, 5.0))
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
