"""ftrainGemmNoAlloc: ftrainGemm with split-k partial tiles in the library's
fixed device scratch array, so no call allocates device memory.

Checked through the C ABI against ftrainGemm on the same inputs: two calls in
a row, the second with a smaller problem (the array keeps the first call's
contents), on shapes whose Primitive 0 is split-k (the scratch is used) and
one whose Primitive 0 is whole-k.  When both entry points run the same
Primitive the results are bit-identical; otherwise both meet the tolerance
against the fp64 oracle.  A problem whose split-k partials exceed the array
runs the first Primitive that fits.
"""

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def capi():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible device")
    from flash_train import capi as c

    return c


def rnd(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g)


def run_both(capi, oracle, m, n, k, seed, with_c):
    a, b = rnd((m, k), seed).cuda(), rnd((k, n), seed + 1).cuda()
    c = rnd((m, n), seed + 2).cuda() if with_c else None
    alpha, beta = 1.25, (0.5 if with_c else 0.0)
    al, be = capi.HostScalar(alpha), capi.HostScalar(beta)
    d_ref = torch.full((m, n), float("nan"), device="cuda")
    d_new = torch.full((m, n), float("nan"), device="cuda")
    cv = capi.matrix(c, [m, n])
    s = torch.cuda.current_stream().cuda_stream
    st = capi.gemm_status(capi.matrix(a), capi.matrix(b), cv, capi.matrix(d_ref), al.view, be.view, stream=s)
    assert st == capi.SUCCESS, capi.last_message()
    st = capi.gemm_no_alloc_status(capi.matrix(a), capi.matrix(b), cv, capi.matrix(d_new), al.view, be.view,
                                   stream=s)
    assert st == capi.SUCCESS, capi.last_message()
    torch.cuda.synchronize()
    ref = oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), None if c is None else c.cpu().numpy(), alpha, beta)
    for name, d in (("ftrainGemm", d_ref), ("ftrainGemmNoAlloc", d_new)):
        rep = oracle.tolerance_check(d.cpu().numpy(), ref, k)
        assert rep["ok"], (name, m, n, k, rep)
    plan = capi.plan_for(a, b, c, d_ref, alpha, beta)
    return plan.names(), d_ref, d_new


@pytest.mark.parametrize("first,second,with_c", [
    ((64, 4096, 4096), (64, 1024, 2048), False),    # split-k Primitive 0 both times, smaller partials second
    ((256, 256, 65536), (128, 128, 16384), True),   # deep k with c
    ((4096, 64, 4096), (1024, 64, 1024), False),
])
def test_no_alloc_matches_ftrain_gemm_on_two_calls(capi, oracle, first, second, with_c):
    for seed, (m, n, k) in ((11, first), (23, second)):
        names, d_ref, d_new = run_both(capi, oracle, m, n, k, seed, with_c)
        if (m, n, k) == first:
            assert names[0].endswith(("_SplitK", "_DeepK")), names  # the scratch array is exercised
        # Same Primitive (its partials fit the array): the same kernels, bit for bit.
        assert torch.equal(d_ref, d_new), (names[0], m, n, k, (d_ref - d_new).abs().max().item())


def test_no_alloc_whole_k_and_odd_shapes(capi, oracle):
    for seed, (m, n, k) in ((5, (1024, 1024, 1024)), (6, (127, 97, 33))):
        names, d_ref, d_new = run_both(capi, oracle, m, n, k, seed, True)
        assert torch.equal(d_ref, d_new), (names[0], m, n, k)


def test_no_alloc_when_partials_exceed_the_scratch(capi, oracle):
    # 4608 x 4608 fp32 is 81 MiB per partial slice: no split-k Primitive fits
    # the 64 MiB array, so ftrainGemmNoAlloc runs the best whole-k Primitive
    # (both results are checked against the oracle in run_both).
    run_both(capi, oracle, 4608, 4608, 2048, 41, False)
