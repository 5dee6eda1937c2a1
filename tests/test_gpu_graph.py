"""Plans inside HIP graphs and across streams, called through the C ABI.

Every execution of a Plan is kernel launches only: split-k partial tiles go
to the caller's workspace or to the buffer Primitive 0 got at Plan creation,
and a grouped Plan's parameter table is uploaded at Plan creation.  So any
execution, the first included, can be captured into a HIP graph and
replayed.  Every replay here runs after the inputs were changed eagerly,
with eager work and synchronisations between replays, and its d is compared
with the fp64 oracle on the new inputs, so a replay that reused stale
results, a stale table or freed memory fails.
"""

import numpy as np
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


@pytest.mark.parametrize("shape,want,workspace,warm", [
    ((1024, 1024, 1024), "", False, True),
    ((64, 4096, 4096), "_DeepK", True, True),      # partials in the caller's workspace (counters cleared first)
    ((64, 4096, 4096), "_DeepK", False, False),    # partials in the Plan's own buffer, first execution captured
    ((64, 1024, 16384), "_SplitK", True, True),    # the split-k kernel + reduction pair
    ((64, 1024, 16384), "_SplitK", False, False),
])
def test_plan_replays_in_a_hip_graph(capi, oracle, shape, want, workspace, warm):
    m, n, k = shape
    a, b, c = rnd((m, k), 1).cuda(), rnd((k, n), 2).cuda(), rnd((m, n), 3).cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, c, d, 1.5, -0.5)
    name = plan.name(0)
    idx = next((i for i, nm in enumerate(plan.names()) if nm.endswith(want)), None) if want else 0
    assert idx is not None, plan.names()
    name = plan.name(idx)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    wsa = (ws.data_ptr(), ws.numel()) if workspace else (0, 0)
    side = torch.cuda.Stream()
    if warm:
        with torch.cuda.stream(side):
            plan.execute(idx, side.cuda_stream, *wsa)  # warm-up outside the capture
        torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        plan.execute(idx, side.cuda_stream, *wsa)
    for rep in range(3):
        a.copy_(rnd((m, k), 10 + rep).cuda())
        d.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), c.cpu().numpy(), 1.5, -0.5)
        rep_ = oracle.tolerance_check(d.cpu().numpy(), ref, k)
        assert rep_["ok"], (name, rep, rep_)


def grouped_plan(capi, G=3, k=64, n=96):
    m_list = [48, 0, 80][:G]
    M = sum(m_list)
    a = rnd((M, k), 4).cuda()
    b = rnd((G * k, n), 5).cuda()
    d = torch.full((M, n), float("nan"), device="cuda")
    ops = capi.GroupedOps("abcd")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    dims = [(m, n) for m in m_list]
    keep = (al, be)
    args = ops.args(a=capi.GroupedSpec(capi.matrix(a), G, dims=[(m, k) for m in m_list]),
                    b=capi.GroupedSpec(capi.matrix(b, [k, n]), G),
                    c=capi.GroupedSpec(capi.View(None, [M, n]), G, dims=dims),
                    d=capi.GroupedSpec(capi.matrix(d), G, dims=dims), alpha=al.view, beta=be.view)
    plan = args.plan()
    args.close()
    return plan, a, b, d, m_list, k, (ops, keep)


def check_grouped(oracle, a, b, d, m_list, k, what):
    a_h, b_h, d_h, row = a.cpu().numpy(), b.cpu().numpy(), d.cpu().numpy(), 0
    for g, m in enumerate(m_list):
        ref = oracle.gemm_f64(a_h[row:row + m], b_h[g * k:(g + 1) * k], None, 1.0, 0.0)
        rep = oracle.tolerance_check(d_h[row:row + m], ref, k)
        assert rep["ok"], (what, g, rep)
        row += m


def test_grouped_plan_on_a_second_stream(capi, oracle):
    plan, a, b, d, m_list, k, keep = grouped_plan(capi)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    plan.execute(0, s1.cuda_stream)
    s1.synchronize()
    check_grouped(oracle, a, b, d, m_list, k, "first stream")
    d.fill_(float("nan"))
    torch.cuda.synchronize()
    plan.execute(0, s2.cuda_stream)
    s2.synchronize()
    check_grouped(oracle, a, b, d, m_list, k, "second stream")


def test_grouped_plan_first_execution_is_captured(capi, oracle):
    plan, a, b, d, m_list, k, keep = grouped_plan(capi)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        plan.execute(0, side.cuda_stream)
    for rep in range(3):
        a.copy_(rnd(tuple(a.shape), 20 + rep).cuda())
        d.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check_grouped(oracle, a, b, d, m_list, k, ("replay", rep))


def test_convenience_graph_survives_plan_cache_eviction(capi, oracle):
    """ftrainGemm keeps up to 32 Plans per thread and destroys the least
    recently used one beyond that.  A Plan it executed under capture is kept
    instead: the graph's split-k kernels point at that Plan's partial buffer.
    Warm up and capture on one stream, evict with 40 other problems, replay."""
    m, n, k = 64, 4096, 4096
    a, b = rnd((m, k), 31).cuda(), rnd((k, n), 32).cuda()
    d = torch.empty(m, n, device="cuda")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    views = (capi.matrix(a), capi.matrix(b), capi.matrix(None, [m, n]), capi.matrix(d), al.view, be.view)
    side = torch.cuda.Stream()
    assert capi.gemm_status(*views, stream=side.cuda_stream) == capi.SUCCESS  # warm-up: creates the cached Plan
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        assert capi.gemm_status(*views, stream=side.cuda_stream) == capi.SUCCESS
    # 40 other problems on the same thread and stream push the captured Plan out of the cache.
    for i in range(40):
        mm = 8 + i
        x, y, z = torch.ones(mm, 32, device="cuda"), torch.ones(32, 16, device="cuda"), torch.empty(mm, 16, device="cuda")
        v = (capi.matrix(x), capi.matrix(y), capi.matrix(None, [mm, 16]), capi.matrix(z), al.view, be.view)
        assert capi.gemm_status(*v, stream=side.cuda_stream) == capi.SUCCESS
    side.synchronize()
    # Memory freed by an evicted Plan would now be handed out again: fill some.
    junk = [torch.full((1 << 20,), 7.0, device="cuda") for _ in range(8)]
    for rep in range(3):
        a.copy_(rnd((m, k), 40 + rep).cuda())
        d.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), None, 1.0, 0.0)
        rep_ = oracle.tolerance_check(d.cpu().numpy(), ref, k)
        assert rep_["ok"], (rep, rep_)
    del junk


def test_captured_convenience_plan_lives_exactly_as_long_as_its_graph(capi, oracle):
    """A Plan that ftrainGemm ran under capture is owned by the capturing
    graph (a HIP user object) as well as by the thread's Plan cache.  Evicted
    from the cache, it stays alive while the graph exists -- the replays after
    the eviction are checked against the oracle -- and is destroyed once the
    graph is.  Counted through the testing library's hook, so every call here
    goes through that library."""
    import gc

    t = capi.testing_lib()
    m, n, k = 64, 4096, 4096
    a, b = rnd((m, k), 51).cuda(), rnd((k, n), 52).cuda()
    d = torch.empty(m, n, device="cuda")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    views = (capi.matrix(a), capi.matrix(b), capi.matrix(None, [m, n]), capi.matrix(d), al.view, be.view)
    side = torch.cuda.Stream()
    assert capi.gemm_status(*views, stream=side.cuda_stream, l=t) == capi.SUCCESS, capi.last_message(t)
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        assert capi.gemm_status(*views, stream=side.cuda_stream, l=t) == capi.SUCCESS
    others = []
    for i in range(40):
        mm = 8 + i
        x, y, z = torch.ones(mm, 32, device="cuda"), torch.ones(32, 16, device="cuda"), torch.empty(mm, 16, device="cuda")
        others.append((x, y, z))
        v = (capi.matrix(x), capi.matrix(y), capi.matrix(None, [mm, 16]), capi.matrix(z), al.view, be.view)
        assert capi.gemm_status(*v, stream=side.cuda_stream, l=t) == capi.SUCCESS
    side.synchronize()
    alive_with_graph = t.ftrainTestingConveniencePlansAlive()
    assert alive_with_graph >= 33, alive_with_graph  # 32 cached + the evicted, captured one
    junk = [torch.full((1 << 20,), 7.0, device="cuda") for _ in range(8)]
    for rep in range(3):
        a.copy_(rnd((m, k), 60 + rep).cuda())
        d.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), None, 1.0, 0.0)
        rep_ = oracle.tolerance_check(d.cpu().numpy(), ref, k)
        assert rep_["ok"], (rep, rep_)
    assert t.ftrainTestingConveniencePlansAlive() == alive_with_graph
    del graph, junk
    gc.collect()
    torch.cuda.synchronize()
    assert t.ftrainTestingConveniencePlansAlive() == alive_with_graph - 1


def test_first_convenience_call_of_a_shape_can_be_captured(capi, oracle):
    """ftrainGemm on a problem it has never seen, inside a global-mode
    capture: Plan preparation would allocate, so the Plan is made without it
    and runs its first Primitive that needs no workspace.  The graph replays
    correctly after the inputs change, and owning it alone, the Plan goes
    when the graph goes."""
    import gc

    t = capi.testing_lib()
    m, n, k = 64, 2048, 8192  # split-k / deep-k is Primitive 0 of this shape
    a, b, c = rnd((m, k), 71).cuda(), rnd((k, n), 72).cuda(), rnd((m, n), 73).cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, c, d, 0.75, 0.5)
    assert plan.name(0).endswith(("_SplitK", "_DeepK")), plan.names()
    al, be = capi.HostScalar(0.75), capi.HostScalar(0.5)
    views = (capi.matrix(a), capi.matrix(b), capi.matrix(c), capi.matrix(d), al.view, be.view)
    side = torch.cuda.Stream()
    before = t.ftrainTestingConveniencePlansAlive()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        st = capi.gemm_status(*views, stream=side.cuda_stream, l=t)
    assert st == capi.SUCCESS, capi.last_message(t)
    assert t.ftrainTestingConveniencePlansAlive() == before + 1
    for rep in range(3):
        a.copy_(rnd((m, k), 80 + rep).cuda())
        d.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), c.cpu().numpy(), 0.75, 0.5)
        rep_ = oracle.tolerance_check(d.cpu().numpy(), ref, k)
        assert rep_["ok"], (rep, rep_)
    del graph
    gc.collect()
    torch.cuda.synchronize()
    assert t.ftrainTestingConveniencePlansAlive() == before


# A child process: the Primitive allow-list is read once per process.
CAPTURE_CHILD = r"""
import json, sys, torch
sys.path[:0] = sys.argv[1:3]
from flash_train import capi
m, n, k = 64, 4096, 4096
g = torch.Generator().manual_seed(5)
a, b = torch.randn(m, k, generator=g).cuda(), torch.randn(k, n, generator=g).cuda()
d = torch.empty(m, n, device="cuda")
al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
views = (capi.matrix(a), capi.matrix(b), capi.matrix(None, [m, n]), capi.matrix(d), al.view, be.view)
side = torch.cuda.Stream()
out = {}
graph = torch.cuda.CUDAGraph()
try:
    with torch.cuda.graph(graph, stream=side):
        out["status"] = capi.gemm_status(*views, stream=side.cuda_stream)
        out["message"] = capi.last_message()
except Exception as e:  # an empty capture may be refused by torch; the status is what is checked
    out["capture_error"] = str(e)[:200]
print("RESULT " + json.dumps(out))
"""


def test_uncached_capture_without_a_fitting_primitive_is_unsupported():
    """Under capture, a first ftrainGemm call whose every Primitive needs a
    workspace (the allow-list keeps split-k Primitives only) and gets none
    returns UNSUPPORTED and names the ways out, instead of allocating."""
    import json
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, FTRAIN_ENABLED_PRIMITIVES="Fp32Mfma16Gemm_64x128_Dma_SplitK,Fp32Mfma16Gemm_64x64_Dma_SplitK")
    proc = subprocess.run([sys.executable, "-c", CAPTURE_CHILD, os.path.join(repo, "flash-train_amd"), repo],
                          env=env, capture_output=True, text=True, timeout=110)
    assert proc.returncode == 0, proc.stderr[-2000:]
    out = json.loads(next(x for x in proc.stdout.splitlines() if x.startswith("RESULT "))[len("RESULT "):])
    assert out["status"] == 4, out  # UNSUPPORTED
    assert "stream capture" in out["message"] and "ftrainGemmNoAlloc" in out["message"], out
