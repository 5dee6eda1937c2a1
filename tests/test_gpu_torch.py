"""flash_train.torch.gemm on the device.

Mirrors the reference's binding test (tests/python/torch_gemm_test.py:15-71):
the same shape grid, seed and tolerances against torch's own formula, the
no-c and default-argument cases, and the RuntimeError cases.  Adds an fp64
oracle check, current-stream ordering, in-place aliasing and NaN propagation.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SHAPE_GRID = [(1, 1, 1), (3, 4, 2), (16, 16, 16), (64, 48, 32), (129, 65, 17), (33, 257, 65), (256, 128, 64)]


@pytest.fixture(scope="module")
def ft():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible device")
    import flash_train.torch as m

    return m


def make_inputs(shape=(128, 64, 96)):
    generator = torch.Generator(device="cuda").manual_seed(7)
    m, k, n = shape
    a = torch.randn(m, k, device="cuda", generator=generator)
    b = torch.randn(k, n, device="cuda", generator=generator)
    c = torch.randn(m, n, device="cuda", generator=generator)
    return a, b, c


@pytest.mark.parametrize("shape", SHAPE_GRID)
def test_gemm_matches_matmul(ft, shape):
    a, b, c = make_inputs(shape)
    d = ft.gemm(a, b, c, alpha=1.5, beta=0.25)
    torch.testing.assert_close(d, 1.5 * (a @ b) + 0.25 * c, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("shape", SHAPE_GRID + [(8192, 1024, 64), (1, 8192, 4096)])
def test_gemm_matches_fp64_oracle(ft, oracle, shape):
    a, b, c = make_inputs(shape)
    d = ft.gemm(a, b, c, alpha=1.5, beta=0.25)
    ref = oracle.gemm_f64(a.cpu(), b.cpu(), c.cpu(), 1.5, 0.25)
    rep = oracle.tolerance_check(d.cpu().numpy(), ref, shape[1])
    assert rep["ok"], rep


def test_gemm_without_c(ft):
    a, b, _ = make_inputs()
    torch.testing.assert_close(ft.gemm(a, b, alpha=1.5), 1.5 * (a @ b), rtol=1e-4, atol=1e-3)


def test_gemm_defaults(ft):
    a, b, _ = make_inputs()
    torch.testing.assert_close(ft.gemm(a, b), a @ b, rtol=1e-4, atol=1e-3)


def test_rejects_shape_mismatch(ft):
    a, _, _ = make_inputs()
    with pytest.raises(RuntimeError):
        ft.gemm(a, torch.randn(3, 3, device="cuda"))
    with pytest.raises(RuntimeError):
        ft.gemm(a, torch.randn(64, 96, device="cuda"), torch.randn(5, 5, device="cuda"))


def test_rejects_cpu_tensor(ft):
    a, b, _ = make_inputs()
    with pytest.raises(RuntimeError):
        ft.gemm(a.cpu(), b)


def test_rejects_float64(ft):
    a, b, _ = make_inputs()
    with pytest.raises(RuntimeError):
        ft.gemm(a.to(torch.float64), b)


def test_rejects_non_contiguous_and_wrong_rank(ft):
    a, b, _ = make_inputs()
    with pytest.raises(RuntimeError):
        ft.gemm(a.t(), b.t())
    with pytest.raises(RuntimeError):
        ft.gemm(a.reshape(-1), b)


def test_runs_on_the_current_stream(ft):
    a, b, c = make_inputs((512, 512, 512))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        x = a * 2.0  # produced on s; the GEMM must be ordered after it
        d = ft.gemm(x, b, c, alpha=1.0, beta=1.0)
        e = d + 1.0
    s.synchronize()
    torch.testing.assert_close(e, (2.0 * a) @ b + c + 1.0, rtol=1e-4, atol=1e-3)


def test_nan_propagates_from_c_even_with_zero_beta(ft):
    a, b, c = make_inputs((64, 64, 64))
    c[3, 4] = float("nan")
    d = ft.gemm(a, b, c, alpha=1.0, beta=0.0)
    assert torch.isnan(d[3, 4]) and torch.isfinite(d).sum() == d.numel() - 1
