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


def test_no_alloc_first_call_allocates_nothing_and_can_be_captured(capi, oracle):
    """The first ftrainGemmNoAlloc call of a shape creates its Plan: free
    device memory is the same before and after it (warm-up calls on other
    shapes have loaded the kernels' code and looked up the scratch array), and
    the first call of yet another shape can run inside a global-mode capture,
    whose replays are checked against the oracle after the inputs change."""
    s = torch.cuda.current_stream().cuda_stream
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)

    def call(m, n, k, seed, stream=s):
        a, b = rnd((m, k), seed).cuda(), rnd((k, n), seed + 1).cuda()
        d = torch.full((m, n), float("nan"), device="cuda")
        views = (capi.matrix(a), capi.matrix(b), capi.matrix(None, [m, n]), capi.matrix(d), al.view, be.view)
        return a, b, d, views

    for seed, shape in ((91, (64, 4096, 4096)), (93, (4096, 64, 4096)), (95, (256, 256, 65536))):
        *_, views = call(*shape, seed)
        assert capi.gemm_no_alloc_status(*views, stream=s) == capi.SUCCESS, capi.last_message()
    torch.cuda.synchronize()
    a, b, d, views = call(64, 3072, 4096, 97)
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    assert capi.gemm_no_alloc_status(*views, stream=s) == capi.SUCCESS, capi.last_message()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free_before
    rep = oracle.tolerance_check(d.cpu().numpy(), oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), None, 1.0, 0.0),
                                 4096)
    assert rep["ok"], rep

    m, n, k = 64, 2560, 8192
    side = torch.cuda.Stream()
    a, b, d, views = call(m, n, k, 99, side.cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        st = capi.gemm_no_alloc_status(*views, stream=side.cuda_stream)
    assert st == capi.SUCCESS, capi.last_message()
    for rep_i in range(3):
        a.copy_(rnd((m, k), 100 + rep_i).cuda())
        d.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), None, 1.0, 0.0)
        rep = oracle.tolerance_check(d.cpu().numpy(), ref, k)
        assert rep["ok"], (rep_i, rep)
    del graph


# Run in a child process: the Primitive allow-list is read once per process.
FALLBACK_CHILD = r"""
import json, sys, torch
sys.path[:0] = sys.argv[1:3]
from flash_train import capi
from oracle import oracle
m, n, k = 4608, 4608, 2048
g = torch.Generator().manual_seed(41)
a, b = torch.randn(m, k, generator=g).cuda(), torch.randn(k, n, generator=g).cuda()
d_plan = torch.full((m, n), float("nan"), device="cuda")
d_new = torch.full((m, n), float("nan"), device="cuda")
plan = capi.plan_for(a, b, None, d_plan, 1.0, 0.0)
names = plan.names()
s = torch.cuda.current_stream().cuda_stream
if len(names) > 1:
    plan.execute(1, s)
al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
st = capi.gemm_no_alloc_status(capi.matrix(a), capi.matrix(b), capi.matrix(None, [m, n]), capi.matrix(d_new),
                               al.view, be.view, stream=s)
msg = capi.last_message()
torch.cuda.synchronize()
out = {"names": names, "status": st, "message": msg}
if st == capi.SUCCESS:
    out["equal_to_primitive_1"] = bool(torch.equal(d_plan, d_new))
    rows = list(range(0, m, 97))
    ref = oracle.gemm_f64(a.cpu().numpy()[rows], b.cpu().numpy(), None, 1.0, 0.0)
    out["ok"] = bool(oracle.tolerance_check(d_new.cpu().numpy()[rows], ref, k)["ok"])
print("RESULT " + json.dumps(out))
"""


def run_fallback_child(enabled):
    import json
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, FTRAIN_ENABLED_PRIMITIVES=enabled)
    proc = subprocess.run([sys.executable, "-c", FALLBACK_CHILD, os.path.join(repo, "flash-train_amd"), repo],
                          env=env, capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, proc.stderr[-2000:]
    line = next(x for x in proc.stdout.splitlines() if x.startswith("RESULT "))
    return json.loads(line[len("RESULT "):])


def test_no_alloc_when_partials_exceed_the_scratch():
    # 4608 x 4608 fp32 is 81 MiB per partial slice, more than the 64 MiB
    # array.  With a split-k Primitive ranked first (the allow-list keeps it
    # and the SIMT kernel only), ftrainGemmNoAlloc runs Primitive 1, bit for
    # bit as the Plan's own Primitive 1 does.
    out = run_fallback_child("Fp32Mfma16Gemm_128x128_Dma_SplitK,Fp32Gemm")
    assert out["names"] == ["Fp32Mfma16Gemm_128x128_Dma_SplitK", "Fp32Gemm"], out
    assert out["status"] == 0, out
    assert out["equal_to_primitive_1"] and out["ok"], out


def test_no_alloc_rejects_a_plan_without_a_fitting_primitive():
    out = run_fallback_child("Fp32Mfma16Gemm_128x128_Dma_SplitK")
    assert out["names"] == ["Fp32Mfma16Gemm_128x128_Dma_SplitK"], out
    assert out["status"] == 4, out  # UNSUPPORTED
    assert "device scratch array" in out["message"] and "Fp32Mfma16Gemm_128x128_Dma_SplitK" in out["message"], out
