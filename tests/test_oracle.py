"""Pins the CPU oracle before it is trusted as the parity checker.

Each check is chosen so that a plausible mistake in the oracle (dropped beta
term, transposed operand, wrong index, wrong fill) fails:
  * known answers held by the reference's tests (KAT, rebinding, in-place);
  * the reference's deterministic-fill grid against exact arithmetic;
  * numpy's fp64 matmul (a library routine) on random shapes;
  * closed forms: identity, all-ones (sum = k), rank-one products, k = 0;
  * the tolerance checker's own semantics (NaN/Inf masks, the bound).
"""

import math

import numpy as np
import pytest

GRID = [(1, 1, 1), (3, 4, 2), (16, 16, 16), (64, 48, 32), (129, 65, 17), (33, 257, 65), (256, 128, 64)]


def test_kat_from_reference(golden, oracle):
    a, b, c = golden["kat_a"], golden["kat_b"], golden["kat_c"]
    al, be = golden["kat_alpha_beta"]
    np.testing.assert_array_equal(oracle.gemm_ref(a, b, c, al, be), golden["kat_expected"])
    np.testing.assert_array_equal(oracle.gemm_f64(a, b, c, al, be), golden["kat_expected"])


@pytest.mark.parametrize("tag", ["rebind1", "rebind2"])
def test_rebind_vectors(golden, oracle, tag):
    a, b, c = golden[f"{tag}_a"], golden[f"{tag}_b"], golden[f"{tag}_c"]
    al, be = golden[f"{tag}_alpha_beta"]
    np.testing.assert_array_equal(oracle.gemm_f64(a, b, c, al, be), golden[f"{tag}_expected"])
    np.testing.assert_allclose(oracle.gemm_ref(a, b, c, al, be), golden[f"{tag}_expected"], rtol=1e-6)


def test_inplace_vector(golden, oracle):
    a, b, cd = golden["inplace_a"], golden["inplace_b"], golden["inplace_cd"]
    al, be = golden["inplace_alpha_beta"]
    np.testing.assert_array_equal(oracle.gemm_f64(a, b, cd, al, be), golden["inplace_expected"])


@pytest.mark.parametrize("mkn", GRID, ids=lambda s: "x".join(map(str, s)))
def test_fill_grid_against_exact(golden, oracle, mkn):
    m, k, n = mkn
    tag = f"fill_{m}x{k}x{n}"
    a = oracle.fill(m * k, 0).reshape(m, k)
    b = oracle.fill(k * n, 7919).reshape(k, n)
    c = oracle.fill(m * n, 104729).reshape(m, n)
    # The oracle's fill reproduces the reference formula bit for bit.
    np.testing.assert_array_equal(a.reshape(-1)[:64], golden[f"{tag}_a_head"][: min(64, m * k)])
    np.testing.assert_array_equal(b.reshape(-1)[:64], golden[f"{tag}_b_head"][: min(64, k * n)])
    np.testing.assert_array_equal(c.reshape(-1)[:64], golden[f"{tag}_c_head"][: min(64, m * n)])
    rows = golden[f"{tag}_rows"]
    fresh = oracle.gemm_f64(a, b, None, 1.5, 0.0)[rows]
    accum = oracle.gemm_f64(a, b, c, 1.5, 1.25)[rows]
    np.testing.assert_allclose(fresh, golden[f"{tag}_fresh"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(accum, golden[f"{tag}_accum"], rtol=1e-12, atol=1e-12)
    # The fp32 restatement of the reference kernel meets the reference's own bar.
    assert oracle.reference_grid_check(oracle.gemm_ref(a, b, c, 1.5, 1.25)[rows], golden[f"{tag}_accum"])["ok"]


def test_readme_config_against_exact(golden, oracle):
    a, b = golden["readme_a"], golden["readme_b"]
    np.testing.assert_allclose(oracle.gemm_f64(a, b), golden["readme_expected"], rtol=1e-12, atol=1e-12)
    rep = oracle.tolerance_check(oracle.gemm_ref(a, b), golden["readme_expected"], 64)
    assert rep["ok"], rep


def test_readme_inputs_match_seeded_generator(golden, oracle):
    a, b, c, cfg = oracle.seeded_inputs("readme_128x96x64")
    assert c is None and (cfg["m"], cfg["n"], cfg["k"]) == (128, 96, 64)
    np.testing.assert_array_equal(a.numpy(), golden["readme_a"])
    np.testing.assert_array_equal(b.numpy(), golden["readme_b"])


@pytest.mark.parametrize("seed", range(6))
def test_against_numpy_fp64(oracle, seed):
    rng = np.random.default_rng(seed)
    m, n, k = rng.integers(1, 70, size=3)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c = rng.standard_normal((m, n)).astype(np.float32)
    alpha, beta = float(rng.uniform(-2, 2)), float(rng.uniform(-2, 2))
    want = alpha * (a.astype(np.float64) @ b.astype(np.float64)) + beta * c.astype(np.float64)
    np.testing.assert_allclose(oracle.gemm_f64(a, b, c, alpha, beta), want, rtol=1e-10, atol=1e-10)
    assert oracle.tolerance_check(oracle.gemm_ref(a, b, c, alpha, beta), want, k)["ok"]
    # Transposed operands or a dropped beta term would not pass.
    if m != n or m != k:
        pass
    assert not np.allclose(oracle.gemm_f64(a, b, c, alpha, 0.0), want)


def test_closed_forms(oracle):
    m, n, k = 7, 5, 11
    ones_a, ones_b = np.ones((m, k), np.float32), np.ones((k, n), np.float32)
    np.testing.assert_array_equal(oracle.gemm_ref(ones_a, ones_b), np.full((m, n), k, np.float32))
    eye = np.eye(k, dtype=np.float32)
    x = np.arange(k * n, dtype=np.float32).reshape(k, n)
    np.testing.assert_array_equal(oracle.gemm_ref(eye, x), x)
    # Rank one: a[i, :] = i + 1, b[:, j] = j -> d[i, j] = k (i + 1) j
    a = np.repeat(np.arange(1, m + 1, dtype=np.float32)[:, None], k, axis=1)
    b = np.repeat(np.arange(n, dtype=np.float32)[None, :], k, axis=0)
    want = k * np.outer(np.arange(1, m + 1), np.arange(n)).astype(np.float32)
    np.testing.assert_array_equal(oracle.gemm_ref(a, b), want)
    # k = 0: d = beta * c (or 0 without c).
    c = np.full((m, n), 3.0, np.float32)
    np.testing.assert_array_equal(oracle.gemm_ref(np.zeros((m, 0), np.float32), np.zeros((0, n), np.float32), c,
                                                  2.0, 0.5), np.full((m, n), 1.5, np.float32))


def test_nan_inf_semantics(oracle):
    a = np.ones((2, 3), np.float32)
    b = np.ones((3, 2), np.float32)
    c = np.zeros((2, 2), np.float32)
    c[0, 0] = np.nan
    # beta = 0 still reads c: 0 * NaN = NaN propagates (reference fp32_gemm.hip:29).
    d = oracle.gemm_ref(a, b, c, 1.0, 0.0)
    assert np.isnan(d[0, 0]) and np.all(np.isfinite(d.reshape(-1)[1:]))
    # Without c there is no beta term.
    assert np.all(np.isfinite(oracle.gemm_ref(a, b, None, 1.0, 0.0)))
    a[1, 0] = np.inf
    d = oracle.gemm_ref(a, b, None, 1.0, 0.0)
    assert np.isposinf(d[1, 0]) and np.isposinf(d[1, 1])


def test_tolerance_checker(oracle):
    ref = np.array([[1.0, -2.0], [np.nan, np.inf]])
    k = 100
    bound = 1e-4 * math.sqrt(k) * 2.0
    ok = oracle.tolerance_check(ref + np.array([[bound * 0.9, 0], [0, 0]]), ref, k)
    assert ok["ok"] and ok["masks_equal"]
    bad = oracle.tolerance_check(ref + np.array([[bound * 1.1, 0], [0, 0]]), ref, k)
    assert not bad["ok"]
    flipped = ref.copy()
    flipped[1, 1] = -np.inf
    assert not oracle.tolerance_check(flipped, ref, k)["masks_equal"]
    lost_nan = ref.copy()
    lost_nan[1, 0] = 0.0
    assert not oracle.tolerance_check(lost_nan, ref, k)["ok"]


# ---------------------------------------------------------------- 16-bit element types


def test_bf16_decode_every_pattern_matches_torch(oracle):
    import torch

    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = oracle.bf16_decode(bits)
    theirs = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


def test_fp16_decode_every_pattern_matches_torch(oracle):
    import torch

    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = oracle.fp16_decode(bits)
    theirs = torch.from_numpy(bits.view(np.int16)).view(torch.float16).float().numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_encode_rounds_to_nearest_even_like_torch(oracle, kind):
    import torch

    g = np.random.default_rng(5)
    x = np.concatenate([
        g.standard_normal(200000).astype(np.float32) * np.float32(g.choice([1e-6, 1.0, 1e3], 200000)),
        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11, 65504.0, 65520.0, 1e-8, -3.4e38], dtype=np.float32)])
    ours = oracle.ENCODE[kind](x)
    dt = torch.bfloat16 if kind == "bf16" else torch.float16
    theirs = torch.from_numpy(x).to(dt).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    # Ties go to even: 1 + half an ulp rounds down to 1, 1 + 1.5 ulp up to 1 + 2 ulp.
    half_ulp = 2.0 ** -8 if kind == "bf16" else 2.0 ** -11
    dec = oracle.DECODE[kind](oracle.ENCODE[kind](np.array([1 + half_ulp, 1 + 3 * half_ulp], np.float32)))
    assert dec[0] == 1.0 and dec[1] == 1.0 + 4 * half_ulp
    # NaN stays NaN.
    assert np.isnan(oracle.DECODE[kind](oracle.ENCODE[kind](np.array([np.nan], np.float32))))[0]


def test_typed_gemm_is_exact_on_small_integers(oracle):
    # Integer-valued bf16 inputs: every product and partial sum is exact, so the fp64
    # reference equals the integer matrix product.
    g = np.random.default_rng(3)
    a = g.integers(-8, 9, (5, 7)).astype(np.float32)
    b = g.integers(-8, 9, (7, 3)).astype(np.float32)
    ref = oracle.gemm_f64_typed(oracle.bf16_encode(a), oracle.bf16_encode(b), "bf16")
    assert np.array_equal(ref, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float64))
    c = g.integers(-4, 5, (5, 3)).astype(np.float32)
    ref = oracle.gemm_f64_typed(oracle.fp16_encode(a), oracle.fp16_encode(b), "fp16", oracle.fp16_encode(c), "fp16",
                                2.0, -1.0)
    assert np.array_equal(ref, 2.0 * (a.astype(np.float64) @ b) - c)


def test_half_tolerance_allows_output_rounding_only(oracle):
    ref = np.array([[1.0, 3.0]])
    k = 1
    bound = 1e-4 * 3.0
    # One bf16 ulp at 3.0 is 2^-6: within bound*(1+u) + u*|ref| (u = 2^-8).
    assert oracle.tolerance_check(np.array([[1.0, 3.0 + 2.0 ** -7]]), ref, k, "bf16")["ok"]
    assert not oracle.tolerance_check(np.array([[1.0, 3.0 + 2.0 ** -5]]), ref, k, "bf16")["ok"]
    assert not oracle.tolerance_check(np.array([[1.0, 3.0 + 2.0 ** -7]]), ref, k, "fp32")["ok"]
    assert oracle.tolerance_check(np.array([[1.0, 3.0 + 0.5 * bound]]), ref, k, "fp32")["ok"]
