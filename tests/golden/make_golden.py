#!/usr/bin/env python3
"""Writes tests/golden/gemm_golden.npz: known-answer vectors for the GEMM path.

Sources of the vectors (all from the reference's own tests, /root/reference):
  * kat            tests/api/gemm_api_test.cpp:392-438 -- 2*[[1,2],[3,4]]@[[5,6],[7,8]] + 0.5*0
                   = [38, 44, 86, 100] (the literal answer is the reference's).
  * rebind_*       tests/api/gemm_api_test.cpp:27-38 -- two 3x2 @ 2x4 problems with
                   (alpha, beta) = (2, -1) and (1, 0.5).
  * inplace        tests/api/gemm_api_test.cpp:340-343 -- c == d, alpha 2, beta 3.
  * fill_*         tests/api/gemm_numerics_test.cpp:30-32,73-75,92-94,129-137 -- the
                   deterministic fill v(i) = ((i*2654435761) mod 199)/199 - 0.5 in fp32,
                   offsets a +0, b +7919, c +104729, alpha 1.5, beta 0 (null c) and 1.25,
                   over the reference's (m, k, n) grid.
  * readme         BASELINE config 1: a 128x64, b 64x96 ~ N(0,1) from a CPU
                   torch.Generator seeded 2026 (a then b), alpha 1, beta 0, no c.

Expected outputs are computed here independently of the oracle: every fp32
product is exact in fp64, each dot product is summed exactly and rounded once
(math.fsum), and alpha*S + beta*c is formed in exact rational arithmetic
(fractions.Fraction) before one final rounding to fp64.  The fill inputs are
produced with numpy fp32 arithmetic, not with the oracle's C fill.

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import os
from fractions import Fraction

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_golden.npz")
GRID = [(1, 1, 1), (3, 4, 2), (16, 16, 16), (64, 48, 32), (129, 65, 17), (33, 257, 65), (256, 128, 64)]
FULL_LIMIT = 4096  # outputs stored in full up to this many; larger shapes keep a fixed sample


def fill(count: int, offset: int) -> np.ndarray:
    i = (np.arange(count, dtype=np.uint64) + np.uint64(offset))
    q = (i * np.uint64(2654435761)) % np.uint64(199)  # wraps mod 2^64 like the C++ code
    return (q.astype(np.float32) / np.float32(199.0) - np.float32(0.5)).astype(np.float32)


def exact_gemm(a: np.ndarray, b: np.ndarray, c, alpha: float, beta: float, rows=None) -> np.ndarray:
    m, k = a.shape
    n = b.shape[1]
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    rows = range(m) if rows is None else rows
    out = []
    for r in rows:
        line = []
        for col in range(n):
            s = math.fsum(a64[r, :] * b64[:, col])  # fp32*fp32 products are exact in fp64
            v = Fraction(alpha) * Fraction(s)
            if c is not None:
                v += Fraction(beta) * Fraction(float(c[r, col]))
            line.append(float(v))
        out.append(line)
    return np.array(out, dtype=np.float64).reshape(len(list(rows)), n)


def main() -> None:
    data = {}
    # Convenience KAT.
    data["kat_a"] = np.array([[1, 2], [3, 4]], np.float32)
    data["kat_b"] = np.array([[5, 6], [7, 8]], np.float32)
    data["kat_c"] = np.zeros((2, 2), np.float32)
    data["kat_alpha_beta"] = np.array([2.0, 0.5])
    data["kat_expected"] = np.array([[38, 44], [86, 100]], np.float64)  # literal from the reference test

    a1 = np.array([1.0, 2.0, -1.0, 0.5, 3.0, -2.0], np.float32).reshape(3, 2)
    b1 = np.array([1.0, -1.0, 2.0, 0.0, 0.5, 1.0, -2.0, 3.0], np.float32).reshape(2, 4)
    c1 = np.array([1, 1, 1, 1, 0, 0, 0, 0, -1, -1, -1, -1], np.float32).reshape(3, 4)
    a2 = np.array([-1.0, 1.0, 2.0, 2.0, 0.0, 4.0], np.float32).reshape(3, 2)
    b2 = np.array([0.5, 0.5, 0.5, 0.5, 1.0, 2.0, 3.0, 4.0], np.float32).reshape(2, 4)
    c2 = np.full((3, 4), 2.0, np.float32)
    for tag, (a, b, c, al, be) in {"rebind1": (a1, b1, c1, 2.0, -1.0), "rebind2": (a2, b2, c2, 1.0, 0.5)}.items():
        data[f"{tag}_a"], data[f"{tag}_b"], data[f"{tag}_c"] = a, b, c
        data[f"{tag}_alpha_beta"] = np.array([al, be])
        data[f"{tag}_expected"] = exact_gemm(a, b, c, al, be)
    cd = np.array([1.0, -2.0, 3.0, 0.5, -1.5, 2.5, -3.0, 1.0, 0.0, -4.0, 2.0, 1.5], np.float32).reshape(3, 4)
    data["inplace_a"], data["inplace_b"], data["inplace_cd"] = a1, b1, cd
    data["inplace_alpha_beta"] = np.array([2.0, 3.0])
    data["inplace_expected"] = exact_gemm(a1, b1, cd, 2.0, 3.0)

    # Deterministic-fill grid (m, k, n).
    rng = np.random.default_rng(7)
    for (m, k, n) in GRID:
        tag = f"fill_{m}x{k}x{n}"
        a = fill(m * k, 0).reshape(m, k)
        b = fill(k * n, 7919).reshape(k, n)
        c = fill(m * n, 104729).reshape(m, n)
        if m * n <= FULL_LIMIT:
            rows = np.arange(m)
        else:
            rows = np.sort(rng.choice(m, size=max(1, FULL_LIMIT // n), replace=False))
        data[f"{tag}_rows"] = rows.astype(np.int64)
        data[f"{tag}_a_head"] = a.reshape(-1)[:64].copy()
        data[f"{tag}_b_head"] = b.reshape(-1)[:64].copy()
        data[f"{tag}_c_head"] = c.reshape(-1)[:64].copy()
        data[f"{tag}_fresh"] = exact_gemm(a, b, None, 1.5, 0.0, rows)
        data[f"{tag}_accum"] = exact_gemm(a, b, c, 1.5, 1.25, rows)

    # BASELINE config 1 (README sample), seeded torch CPU generator.
    import torch

    g = torch.Generator().manual_seed(2026)
    a = torch.randn(128, 64, generator=g).numpy()
    b = torch.randn(64, 96, generator=g).numpy()
    data["readme_a"], data["readme_b"] = a, b
    data["readme_expected"] = exact_gemm(a, b, None, 1.0, 0.0)

    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main()
