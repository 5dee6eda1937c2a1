"""Plans inside HIP graphs and across streams, called through the C ABI.

A cached Plan's execution is kernel launches only (a split-k Primitive given
the caller's workspace included), so it can be captured into a HIP graph and
replayed.  Every replay here runs after the inputs were changed eagerly, and
its d is compared with the fp64 oracle on the new inputs, so a replay that
reused stale results or a stale parameter table fails.

A grouped Plan uploads its per-group parameter table with a blocking copy on
its first execution: that execution cannot be captured (UNSUPPORTED with a
reason), and any stream may execute the Plan afterwards.
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


@pytest.mark.parametrize("shape,want", [((1024, 1024, 1024), ""), ((64, 4096, 4096), "_SplitK")])
def test_plan_replays_in_a_hip_graph(capi, oracle, shape, want):
    m, n, k = shape
    a, b, c = rnd((m, k), 1).cuda(), rnd((k, n), 2).cuda(), rnd((m, n), 3).cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, c, d, 1.5, -0.5)
    name = plan.name(0)
    assert name.endswith(want) if want else not name.endswith("_SplitK"), plan.names()
    # Split-k Primitives write their partial tiles to the caller's workspace here.
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        plan.execute(0, side.cuda_stream, ws.data_ptr(), ws.numel())  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        plan.execute(0, side.cuda_stream, ws.data_ptr(), ws.numel())
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
    plan.execute(0, s1.cuda_stream)  # uploads the table
    d.fill_(float("nan"))
    torch.cuda.synchronize()
    plan.execute(0, s2.cuda_stream)  # no ordering with s1: the table must already be complete
    s2.synchronize()
    check_grouped(oracle, a, b, d, m_list, k, "second stream")


def test_grouped_plan_capture_after_first_execution(capi, oracle):
    plan, a, b, d, m_list, k, keep = grouped_plan(capi)
    side = torch.cuda.Stream()
    scratch = torch.zeros(16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        scratch.add_(1.0)  # keeps the captured graph non-empty
        status = plan.execute_status(0, side.cuda_stream)
    assert status == capi.UNSUPPORTED, status
    assert "cannot be captured" in capi.last_message()
    plan.execute(0, side.cuda_stream)  # eager first execution
    side.synchronize()
    check_grouped(oracle, a, b, d, m_list, k, "eager")
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
