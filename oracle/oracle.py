"""Python front end of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only to check results or to time the CPU baseline.
The product path (libflash_train.so, flash_train.torch) never touches it.

Contents
  gemm_ref(a, b, c, alpha, beta)   reference-kernel restatement (fp32 in-order k sum),
                                   /root/reference/src/primitive/hygon/gemm/fp32_gemm.hip:18-31
  gemm_f64(a, b, c, alpha, beta)   fp64 reference of the same formula
  fill(count, offset)              the reference tests' deterministic fill,
                                   /root/reference/tests/api/gemm_numerics_test.cpp:30-32
  tolerance_check(d, ref, k)       the north-star bar: max|d - ref| <= 1e-4 * sqrt(k) * max|ref|
                                   over finite entries, and identical NaN / +Inf / -Inf masks
  reference_grid_check(d, ref)     the reference numerics test's bar, |d - ref| <= 2e-5 + 2e-5 |ref|
                                   (/root/reference/tests/api/gemm_numerics_test.cpp:58-59,
                                   tests/support/numerics.hpp:72-101)
  seeded_inputs(config)            BASELINE inputs: one CPU torch.Generator seeded 2026, a, b, c in order
  bf16_decode / bf16_encode        bfloat16 bit patterns <-> fp32 (exact widening; round to nearest
  fp16_decode / fp16_encode        even when narrowing, NaN kept NaN); the same for IEEE binary16
  gemm_f64_typed(...)              gemm_f64 on operands given as 16-bit patterns (decoded exactly)
  tolerance_check(..., out_type)   for a bf16 / fp16 d, the bar widened by that type's rounding:
                                   |d - ref| <= bound * (1 + u) + u * |ref|, u = 2^-8 (bf16) / 2^-11 (fp16)

The 16-bit element types have no reference kernel (the reference's only kernel is
fp32, fp32_gemm.hip:18-31, though its numeric-type enum names both types,
include/flash_train/common.h:38-65); their products are exact in fp32, so the
fp64 reference of the decoded values is the oracle for them too.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        f64p = ctypes.POINTER(ctypes.c_double)
        u64 = ctypes.c_uint64
        l.ft_oracle_gemm_ref.argtypes = [f32p, f32p, f32p, ctypes.c_float, ctypes.c_float, f32p, u64, u64, u64]
        l.ft_oracle_gemm_ref.restype = None
        l.ft_oracle_gemm_f64.argtypes = [f32p, f32p, f32p, ctypes.c_double, ctypes.c_double, f64p, u64, u64, u64]
        l.ft_oracle_gemm_f64.restype = None
        l.ft_oracle_fill.argtypes = [f32p, u64, u64]
        l.ft_oracle_fill.restype = None
        l.ft_oracle_threads.argtypes = []
        l.ft_oracle_threads.restype = ctypes.c_int
        _lib = l
    return _lib


def _f32(x: np.ndarray):
    return x.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _as_f32(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(x, dtype=np.float32)


def gemm_ref(a, b, c=None, alpha: float = 1.0, beta: float = 0.0) -> np.ndarray:
    a, b = _as_f32(a), _as_f32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    cc = _as_f32(c) if c is not None else None
    d = np.empty((m, n), dtype=np.float32)
    lib().ft_oracle_gemm_ref(_f32(a), _f32(b), _f32(cc) if cc is not None else None, alpha, beta, _f32(d), m, n, k)
    return d


def gemm_f64(a, b, c=None, alpha: float = 1.0, beta: float = 0.0) -> np.ndarray:
    a, b = _as_f32(a), _as_f32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    cc = _as_f32(c) if c is not None else None
    d = np.empty((m, n), dtype=np.float64)
    lib().ft_oracle_gemm_f64(_f32(a), _f32(b), _f32(cc) if cc is not None else None, alpha, beta,
                             d.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), m, n, k)
    return d


def fill(count: int, offset: int = 0) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib().ft_oracle_fill(_f32(out), count, offset)
    return out


def threads() -> int:
    return lib().ft_oracle_threads()


def tolerance_check(d, ref, k: int, out_type: str = "fp32") -> dict:
    """North-star parity bar.  Returns a report; report['ok'] is the verdict.

    bound = 1e-4 * sqrt(max(k, 1)) * max|ref| over finite ref entries; every
    entry where both are finite must satisfy |d - ref| <= bound, and the NaN,
    +Inf and -Inf masks of d and ref must be identical.  For a d rounded to
    bf16 / fp16 (`out_type`, d given as decoded values) each entry may
    further differ by that rounding: |d - ref| <= bound * (1 + u) + u * |ref|.
    """
    u = UNIT_ROUNDOFF[out_type]
    d = np.asarray(d, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert d.shape == ref.shape, (d.shape, ref.shape)
    masks_equal = bool(
        np.array_equal(np.isnan(d), np.isnan(ref))
        and np.array_equal(np.isposinf(d), np.isposinf(ref))
        and np.array_equal(np.isneginf(d), np.isneginf(ref)))
    finite = np.isfinite(ref) & np.isfinite(d)
    scale = float(np.max(np.abs(ref[np.isfinite(ref)]))) if np.isfinite(ref).any() else 0.0
    bound = 1e-4 * math.sqrt(max(k, 1)) * scale
    diff = np.abs(d[finite] - ref[finite])
    err = float(np.max(diff)) if finite.any() else 0.0
    if u > 0 and finite.any():
        allowed = bound * (1 + u) + u * np.abs(ref[finite])
        ok = masks_equal and bool(np.all(diff <= allowed))
    else:
        ok = masks_equal and err <= bound
    return {"ok": ok, "max_abs_err": err, "bound": bound, "ratio": (err / bound) if bound > 0 else (0.0 if err == 0 else math.inf),
            "masks_equal": masks_equal, "max_abs_ref": scale}


# ---- 16-bit element types ----

UNIT_ROUNDOFF = {"fp32": 0.0, "bf16": 2.0 ** -8, "fp16": 2.0 ** -11}


def bf16_decode(bits) -> np.ndarray:
    """bfloat16 patterns (uint16) -> fp32: the pattern is the high half of the fp32 word."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_encode(x) -> np.ndarray:
    """fp32 -> bfloat16 patterns, round to nearest even; NaN stays a (quiet) NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    # Adding 0x7FFF plus the lowest kept bit carries into the kept half exactly when the
    # dropped half is above one half, or equal to it with an odd kept half.
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = np.where(nan, (u >> 16) | 0x0040, rounded)
    return out.astype(np.uint16)


def fp16_decode(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def fp16_encode(x) -> np.ndarray:
    """fp32 -> IEEE binary16 patterns (numpy's round-to-nearest-even conversion)."""
    with np.errstate(over="ignore"):  # out-of-range values become +-inf, as IEEE narrowing does
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


DECODE = {"bf16": bf16_decode, "fp16": fp16_decode}
ENCODE = {"bf16": bf16_encode, "fp16": fp16_encode}


def gemm_f64_typed(a_bits, b_bits, in_type: str, c=None, cd_type: str = "fp32", alpha: float = 1.0,
                   beta: float = 0.0) -> np.ndarray:
    """fp64 reference for a, b given as 16-bit patterns of `in_type`; c is fp32 values or
    16-bit patterns of `cd_type`."""
    a = DECODE[in_type](a_bits)
    b = DECODE[in_type](b_bits)
    cc = None if c is None else (DECODE[cd_type](c) if cd_type != "fp32" else np.asarray(c, np.float32))
    return gemm_f64(a, b, cc, alpha, beta)


def reference_grid_check(d, ref, rel: float = 2e-5, abs_: float = 2e-5) -> dict:
    d = np.asarray(d, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    allowed = abs_ + rel * np.abs(ref)
    ratio = float(np.max(np.abs(d - ref) / np.maximum(allowed, 1e-30))) if d.size else 0.0
    return {"ok": ratio <= 1.0, "worst_ratio": ratio}


# ---- BASELINE.json configs (m, n, k) and their input distributions ----

CONFIGS = {
    "readme_128x96x64": dict(m=128, n=96, k=64, dist="normal", std=1.0, alpha=1.0, beta=0.0, with_c=False),
    "square_4096_beta": dict(m=4096, n=4096, k=4096, dist="normal", std=1.0, alpha=1.0, beta=0.5, with_c=True),
    "square_8192": dict(m=8192, n=8192, k=8192, dist="uniform", std=None, alpha=1.0, beta=0.0, with_c=False),
    "mlp_fwd": dict(m=16384, n=14336, k=4096, dist="normal", std=0.02, alpha=1.0, beta=0.0, with_c=False),
    "mlp_dgrad": dict(m=16384, n=4096, k=14336, dist="normal", std=0.02, alpha=1.0, beta=0.0, with_c=False),
    "skinny_64x4096x4096": dict(m=64, n=4096, k=4096, dist="normal", std=1.0, alpha=1.0, beta=0.0, with_c=False),
    "skinny_4096x64x4096": dict(m=4096, n=64, k=4096, dist="normal", std=1.0, alpha=1.0, beta=0.0, with_c=False),
    "splitk_256x256x65536": dict(m=256, n=256, k=65536, dist="normal", std=1.0, alpha=1.0, beta=0.0, with_c=False),
    "gemv_1x8192x8192": dict(m=1, n=8192, k=8192, dist="normal", std=1.0, alpha=1.0, beta=0.0, with_c=False),
    "odd_127x97x33": dict(m=127, n=97, k=33, dist="normal", std=1.0, alpha=1.0, beta=0.0, with_c=False),
}


def seeded_inputs(name: str, seed: int = 2026):
    """CPU torch tensors a (m x k), b (k x n), c (m x n or None) for a config."""
    import torch

    cfg = CONFIGS[name]
    g = torch.Generator().manual_seed(seed)
    m, n, k = cfg["m"], cfg["n"], cfg["k"]

    def draw(*shape):
        if cfg["dist"] == "uniform":
            return torch.rand(*shape, generator=g) * 2.0 - 1.0
        return torch.randn(*shape, generator=g) * cfg["std"]

    a = draw(m, k)
    b = draw(k, n)
    c = draw(m, n) if cfg["with_c"] else None
    return a, b, c, cfg


def sampled_rows_f64(a, b, c, alpha: float, beta: float, rows: np.ndarray) -> np.ndarray:
    """fp64 reference for selected rows only (large configs)."""
    a_sub = _as_f32(a)[rows]
    c_sub = _as_f32(c)[rows] if c is not None else None
    return gemm_f64(a_sub, b, c_sub, alpha, beta)
