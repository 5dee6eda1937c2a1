"""GPU parity of the HIP GEMM path, called through the C ABI.

Mirrors the reference's device tests (tests/api/gemm_api_test.cpp,
tests/api/gemm_numerics_test.cpp) and adds the BASELINE configurations,
every Primitive of each Plan, NaN/Inf propagation and tails.  Every result is
compared with the CPU oracle (oracle/oracle.py) on the same inputs:
  * the reference numerics grid with the reference's own bar,
    |d - ref| <= 2e-5 + 2e-5 |ref| (gemm_numerics_test.cpp:58-59);
  * everything else with the north-star bar,
    max|d - ref| <= 1e-4 * sqrt(k) * max|ref| against fp64, identical NaN/Inf masks.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GRID = [(1, 1, 1), (3, 4, 2), (16, 16, 16), (64, 48, 32), (129, 65, 17), (33, 257, 65), (256, 128, 64)]


@pytest.fixture(scope="module")
def capi():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible device")
    from flash_train import capi as c

    return c


@pytest.fixture(scope="module")
def ops(capi):
    # Roles added in reverse of the engine's order (gemm_staged_fixture.hpp:20-28).
    return capi.GemmOps(order=("d", "beta", "alpha", "c", "b", "a"))


def dev(x):
    return torch.as_tensor(np.ascontiguousarray(x, dtype=np.float32)).cuda()


def run_plan(capi, ops, a, b, c, d, alpha, beta, index=0):
    plan = capi.plan_for(a, b, c, d, alpha, beta, ops)
    plan.execute(index, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return plan


def report(oracle, d, ref, k):
    rep = oracle.tolerance_check(d.cpu().numpy() if hasattr(d, "cpu") else d, ref, k)
    assert rep["ok"], rep
    return rep


# ---------------------------------------------------------------- reference tests


def test_convenience_kat(capi, golden):
    a, b, c = dev(golden["kat_a"]), dev(golden["kat_b"]), dev(golden["kat_c"])
    d = torch.empty(2, 2, device="cuda")
    al, be = capi.HostScalar(2.0), capi.HostScalar(0.5)
    st = capi.gemm_status(capi.matrix(a), capi.matrix(b), capi.matrix(c), capi.matrix(d), al.view, be.view,
                          stream=torch.cuda.current_stream().cuda_stream)
    assert st == capi.SUCCESS, capi.last_message()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(d.cpu().numpy(), golden["kat_expected"])
    # Inconsistent b: INVALID_ARGUMENT, nothing dispatched.
    st = capi.gemm_status(capi.matrix(a), capi.matrix(b, [3, 3]), capi.matrix(c), capi.matrix(d), al.view, be.view)
    assert st == capi.INVALID_ARGUMENT


def test_rebinds_addresses_and_outlives_ops_and_args(capi, golden):
    ops = capi.GemmOps(order=("d", "beta", "alpha", "c", "b", "a"))
    plans, outs = [], []
    for tag in ("rebind1", "rebind2"):
        a, b, c = dev(golden[f"{tag}_a"]), dev(golden[f"{tag}_b"]), dev(golden[f"{tag}_c"])
        d = torch.empty(3, 4, device="cuda")
        al, be = golden[f"{tag}_alpha_beta"]
        plans.append((capi.plan_for(a, b, c, d, float(al), float(be), ops), (a, b, c)))
        outs.append(d)
    for p, _ in plans:
        assert p.workspace_bytes(0) == 0
    ops.close()  # Plans outlive Ops and Args
    s = torch.cuda.current_stream().cuda_stream
    for p, _ in plans:
        p.execute(0, s)
    torch.cuda.synchronize()
    for tag, d in zip(("rebind1", "rebind2"), outs):
        np.testing.assert_allclose(d.cpu().numpy(), golden[f"{tag}_expected"], rtol=1e-6, atol=1e-6)


def test_in_place_c_equals_d(capi, ops, golden):
    a, b = dev(golden["inplace_a"]), dev(golden["inplace_b"])
    cd = dev(golden["inplace_cd"])
    al, be = golden["inplace_alpha_beta"]
    plan = capi.plan_for(a, b, cd, cd, float(al), float(be), ops)
    for i in range(len(plan)):
        cd.copy_(dev(golden["inplace_cd"]))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        np.testing.assert_allclose(cd.cpu().numpy(), golden["inplace_expected"], rtol=1e-6, atol=1e-6,
                                   err_msg=plan.name(i))


def test_empty_output_launches_nothing(capi, ops):
    d = capi.View(None, [0, 4])
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    args = ops.args(capi.View(None, [0, 2]), capi.View(None, [2, 4]), capi.View(None, [0, 4]), d, al.view, be.view)
    plan = args.plan()
    assert plan.workspace_bytes(0) == 0
    plan.execute(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()


def test_overflow_and_invalid_shapes(capi, ops):
    big = (1 << 63) - 1
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    args = ops.args(capi.View(None, [big, big]), capi.View(None, [big, big]), capi.View(None, [big, big]),
                    capi.View(None, [big, big]), al.view, be.view)
    with pytest.raises(capi.FTrainError) as e:
        args.plan()
    assert e.value.status == capi.OVERFLOW
    x = torch.zeros(16, device="cuda")
    p = x.data_ptr()
    for a_dims, b_dims, d_dims in (([6], [2, 4], [3, 4]), ([3, 2], [3, 4], [3, 4]), ([3, 2], [2, 4], [4, 3])):
        args = ops.args(capi.View(p, a_dims), capi.View(p, b_dims), capi.View(p, [3, 4]), capi.View(p, d_dims),
                        al.view, be.view)
        with pytest.raises(capi.FTrainError) as e:
            args.plan()
        assert e.value.status == capi.INVALID_ARGUMENT


def test_unsupported_storage(capi, ops):
    x = torch.zeros(64, device="cuda")
    p = x.data_ptr()
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    args = ops.args(capi.View(p, [3, 2], numeric_type=capi.FP16), capi.View(p, [2, 4]), capi.View(p, [3, 4]),
                    capi.View(p, [3, 4]), al.view, be.view)
    with pytest.raises(capi.FTrainError) as e:
        args.plan()
    assert e.value.status == capi.UNSUPPORTED
    assert "Fp32Gemm" in e.value.message and "an operand is not fp32" in e.value.message
    args = ops.args(capi.View(p, [3, 2], index_type=capi.INDEX_INVALID, strides=[2, 1]), capi.View(p, [2, 4]),
                    capi.View(p, [3, 4]), capi.View(p, [3, 4]), al.view, be.view)
    with pytest.raises(capi.FTrainError) as e:
        args.plan()
    assert e.value.status == capi.UNSUPPORTED
    args = ops.args(capi.View(None, [3, 2]), capi.View(p, [2, 4]), capi.View(p, [3, 4]), capi.View(p, [3, 4]),
                    al.view, be.view)
    with pytest.raises(capi.FTrainError) as e:
        args.plan()
    assert e.value.status == capi.UNSUPPORTED
    args = ops.args(capi.View(p, [3, 2]), capi.View(p, [2, 4]), capi.View(p, [3, 4]), capi.View(p, [3, 4]),
                    al.view, be.view, compute_type=capi.FP64)
    with pytest.raises(capi.FTrainError) as e:
        args.plan()
    assert e.value.status == capi.UNSUPPORTED
    # Misaligned (not 4-byte) address.
    args = ops.args(capi.View(p + 2, [3, 2]), capi.View(p, [2, 4]), capi.View(p, [3, 4]), capi.View(p, [3, 4]),
                    al.view, be.view)
    with pytest.raises(capi.FTrainError) as e:
        args.plan()
    assert e.value.status == capi.UNSUPPORTED and "float-aligned" in e.value.message


def test_device_mismatch(capi):
    """A Plan bound to another device id refuses to execute (plan.cpp:43-48)."""
    t = capi.testing_lib()
    ops = capi.GemmOps(l=t)
    a = torch.ones(4, 4, device="cuda")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    args = ops.args(capi.matrix(a), capi.matrix(a), capi.matrix(None, [4, 4]), capi.matrix(a), al.view, be.view)
    h = ctypes.c_void_p()
    assert t.ftrainTestingPlanCreateOnDevice(ctypes.byref(h), args.handle, torch.cuda.current_device() + 1) == 0
    plan = capi.Plan(h, t)
    st = plan.execute_status(0, torch.cuda.current_stream().cuda_stream)
    assert st == capi.INVALID_ARGUMENT
    assert "calling thread uses device" in capi.last_message(t)
    assert plan.execute_status(len(plan), 0) == capi.INVALID_ARGUMENT


# ---------------------------------------------------------------- numerics grid


@pytest.mark.parametrize("mkn", GRID, ids=lambda s: "x".join(map(str, s)))
def test_reference_numerics_grid_every_primitive(capi, ops, oracle, golden, mkn):
    m, k, n = mkn
    a_h = oracle.fill(m * k, 0).reshape(m, k)
    b_h = oracle.fill(k * n, 7919).reshape(k, n)
    c_h = oracle.fill(m * n, 104729).reshape(m, n)
    a, b, c = dev(a_h), dev(b_h), dev(c_h)
    rows = golden[f"fill_{m}x{k}x{n}_rows"]
    for with_c, beta, key in ((False, 0.0, "fresh"), (True, 1.25, "accum")):
        d = torch.full((m, n), float("nan"), device="cuda")
        plan = capi.plan_for(a, b, c if with_c else None, d, 1.5, beta, ops)
        for i, name in enumerate(plan.names()):
            d.fill_(float("nan"))
            plan.execute(i, torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            got = d.cpu().numpy()[rows]
            rep = oracle.reference_grid_check(got, golden[f"fill_{m}x{k}x{n}_{key}"])
            assert rep["ok"], (name, key, rep)


@pytest.mark.parametrize("shape", [(1, 1, 1), (5, 3, 7), (31, 33, 35), (64, 64, 64), (100, 300, 17),
                                   (129, 257, 65), (257, 129, 520), (8, 1000, 1024), (3, 8192, 260),
                                   (513, 64, 1500), (64, 8, 2048)])
def test_random_shapes_every_primitive(capi, ops, oracle, shape):
    m, n, k = shape
    g = torch.Generator().manual_seed(m * 1000003 + n * 1009 + k)
    a_h, b_h, c_h = (torch.randn(m, k, generator=g), torch.randn(k, n, generator=g), torch.randn(m, n, generator=g))
    ref = oracle.gemm_f64(a_h, b_h, c_h, 0.75, -0.5)
    a, b, c = a_h.cuda(), b_h.cuda(), c_h.cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, c, d, 0.75, -0.5, ops)
    for i, name in enumerate(plan.names()):
        d.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        rep = oracle.tolerance_check(d.cpu().numpy(), ref, k)
        assert rep["ok"], (name, shape, rep)


@pytest.mark.parametrize("m", [33, 4])  # 4 rows: the skinny (GEMV) Primitives too
def test_zero_depth(capi, ops, m):
    n = 20
    c = torch.randn(m, n, device="cuda")
    d = torch.empty(m, n, device="cuda")
    al, be = capi.HostScalar(2.0), capi.HostScalar(0.5)
    args = ops.args(capi.View(None, [m, 0]), capi.View(None, [0, n]), capi.matrix(c), capi.matrix(d), al.view,
                    be.view)
    plan = args.plan()
    for i in range(len(plan)):
        d.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        torch.testing.assert_close(d, 0.5 * c, rtol=0, atol=0)


@pytest.mark.parametrize("m", [70, 6])  # 6 rows: the skinny (GEMV) Primitives too
def test_nan_inf_propagation(capi, ops, oracle, m):
    n, k = 68, 96
    g = torch.Generator().manual_seed(11)
    a_h, b_h, c_h = torch.randn(m, k, generator=g), torch.randn(k, n, generator=g), torch.randn(m, n, generator=g)
    a_h[3, 5] = float("nan")
    a_h[10 % m, 7] = float("inf")
    b_h[9, 40] = float("-inf")
    c_h[50 % m, 50] = float("nan")
    c_h[60 % m, 1] = float("inf")
    for beta in (0.0, 0.5):
        ref = oracle.gemm_f64(a_h, b_h, c_h, 1.0, beta)
        d = torch.empty(m, n, device="cuda")
        plan = capi.plan_for(a_h.cuda(), b_h.cuda(), c_h.cuda(), d, 1.0, beta, ops)
        if m <= 8:
            assert "Fp32Gemv" in plan.names() and "Fp32Gemv_SplitK" in plan.names(), plan.names()
        for i, name in enumerate(plan.names()):
            plan.execute(i, torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            rep = oracle.tolerance_check(d.cpu().numpy(), ref, k)
            assert rep["masks_equal"], (name, beta)
            assert rep["ok"], (name, beta, rep)


# ---------------------------------------------------------------- BASELINE configs


SMALL_CONFIGS = ["readme_128x96x64", "skinny_64x4096x4096", "skinny_4096x64x4096", "splitk_256x256x65536",
                 "gemv_1x8192x8192", "odd_127x97x33"]


@pytest.mark.parametrize("name", SMALL_CONFIGS)
def test_baseline_config_full_check(capi, ops, oracle, name):
    a_h, b_h, c_h, cfg = oracle.seeded_inputs(name)
    ref = oracle.gemm_f64(a_h, b_h, c_h, cfg["alpha"], cfg["beta"])
    d = torch.empty(cfg["m"], cfg["n"], device="cuda")
    plan = capi.plan_for(a_h.cuda(), b_h.cuda(), c_h.cuda() if c_h is not None else None, d, cfg["alpha"],
                         cfg["beta"], ops)
    print(name, plan.names())
    for i, pname in enumerate(plan.names()):
        d.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        rep = oracle.tolerance_check(d.cpu().numpy(), ref, cfg["k"])
        assert rep["ok"], (name, pname, rep)
        # Far inside the bar, not just under it: a dropped or repeated k slice
        # or a misplaced partial tile lands near or above it.
        assert rep["max_abs_err"] <= 1e-2 * rep["bound"], (name, pname, rep)


@pytest.mark.parametrize("name,every", [("square_4096_beta", True), ("square_8192", False), ("mlp_fwd", False),
                                        ("mlp_dgrad", True)])
def test_baseline_config_sampled_rows(capi, ops, oracle, name, every):
    """Large configs: fp64 reference on 64 seeded rows x all columns.  Primitive 0
    everywhere; every Primitive of the Plan on the deepest config (MLP dgrad, k =
    14336) and on the one with c (4096^3, beta 0.5), so a Primitive another box,
    an environment filter or a Finder change could promote is checked at full
    size too.  Each result must also sit far inside the bar (1e-2 of it)."""
    a_h, b_h, c_h, cfg = oracle.seeded_inputs(name)
    rows = np.sort(np.random.default_rng(2026).choice(cfg["m"], size=64, replace=False))
    ref = oracle.sampled_rows_f64(a_h, b_h, c_h, cfg["alpha"], cfg["beta"], rows)
    d = torch.empty(cfg["m"], cfg["n"], device="cuda")
    plan = capi.plan_for(a_h.cuda(), b_h.cuda(), c_h.cuda() if c_h is not None else None, d, cfg["alpha"],
                         cfg["beta"], ops)
    names = plan.names()
    print(name, names)
    for i in (range(len(names)) if every else [0]):
        d.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = d[torch.as_tensor(rows).cuda()].cpu().numpy()
        rep = oracle.tolerance_check(got, ref, cfg["k"])
        assert rep["ok"], (name, names[i], rep)
        assert rep["max_abs_err"] <= 1e-2 * rep["bound"], (name, names[i], rep)
        assert not torch.isnan(d).any().item(), (name, names[i], "left part of d unwritten")
    plan.execute(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    # Size-independent property over the whole output: row sums equal a @ (b @ 1).
    ones = torch.ones(cfg["n"], 1, dtype=torch.float64)
    row_sums = d.double().cpu() @ ones
    want = cfg["alpha"] * (a_h.double() @ (b_h.double() @ ones))
    if c_h is not None:
        want += cfg["beta"] * (c_h.double() @ ones)
    err = (row_sums - want).abs().max().item()
    scale = want.abs().max().item() + np.sqrt(cfg["n"] * cfg["k"])
    assert err <= 1e-4 * np.sqrt(cfg["k"]) * scale, (name, err, scale)


def test_convenience_calls_reuse_plans_without_changing_results(capi, oracle):
    """ftrainGemm keeps recently used Plans; repeated calls must still honour
    new buffer contents, new alpha/beta values and new addresses."""
    m, n, k = 96, 80, 64
    g = torch.Generator().manual_seed(3)
    a_h, b_h, c_h = torch.randn(m, k, generator=g), torch.randn(k, n, generator=g), torch.randn(m, n, generator=g)
    a, b, c = a_h.cuda(), b_h.cuda(), c_h.cuda()
    d = torch.empty(m, n, device="cuda")
    s = torch.cuda.current_stream().cuda_stream

    def call(alpha, beta, dd=d):
        al, be = capi.HostScalar(alpha), capi.HostScalar(beta)
        st = capi.gemm_status(capi.matrix(a), capi.matrix(b), capi.matrix(c), capi.matrix(dd), al.view, be.view,
                              stream=s)
        assert st == capi.SUCCESS, capi.last_message()
        torch.cuda.synchronize()
        return dd.cpu().numpy()

    for alpha, beta in ((1.0, 0.0), (1.0, 0.0), (2.0, 0.5), (1.0, 0.0)):
        rep = oracle.tolerance_check(call(alpha, beta), oracle.gemm_f64(a.cpu(), b.cpu(), c.cpu(), alpha, beta), k)
        assert rep["ok"], (alpha, beta, rep)
    a.mul_(-1.0)  # same addresses, new contents
    rep = oracle.tolerance_check(call(1.0, 0.0), oracle.gemm_f64(a.cpu(), b.cpu(), c.cpu(), 1.0, 0.0), k)
    assert rep["ok"], rep
    d2 = torch.empty(m, n, device="cuda")  # new output address
    rep = oracle.tolerance_check(call(1.0, 1.0, d2), oracle.gemm_f64(a.cpu(), b.cpu(), c.cpu(), 1.0, 1.0), k)
    assert rep["ok"], rep


def test_caller_workspace_is_used_for_split_k(capi, ops, oracle):
    """Workspace contract of split-k Primitives (reference common.h:548-576):
    Primitive 0 owns a partial buffer allocated at Plan creation and requires
    no workspace; every other split Primitive reports its partial bytes, is
    rejected with INVALID_ARGUMENT without them, and runs with them.  Results
    agree either way."""
    m, n, k = 64, 512, 8192
    g = torch.Generator().manual_seed(5)
    a_h, b_h = torch.randn(m, k, generator=g), torch.randn(k, n, generator=g)
    ref = oracle.gemm_f64(a_h, b_h)
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a_h.cuda(), b_h.cuda(), None, d, 1.0, 0.0, ops)
    names = plan.names()
    split = [i for i, nm in enumerate(names) if nm.endswith(("_SplitK", "_DeepK"))]
    assert len(split) >= 2, names
    assert plan.workspace_bytes(0) == 0
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    for i in split:
        need = plan.workspace_bytes(i)
        if i == 0:
            assert need == 0
        else:
            assert need > 16384, (names[i], need)  # arrival counters, then partial tiles
            assert plan.execute_status(i, s) == capi.INVALID_ARGUMENT
            assert "workspace" in capi.last_message()
            assert plan.execute_status(i, s, ws.data_ptr(), need - 1) == capi.INVALID_ARGUMENT
        for workspace in ((0, ws.data_ptr()) if i == 0 else (ws.data_ptr(),)):
            d.fill_(float("nan"))
            assert plan.execute_status(i, s, workspace, ws.numel() if workspace else 0) == capi.SUCCESS
            torch.cuda.synchronize()
            rep = oracle.tolerance_check(d.cpu().numpy(), ref, k)
            assert rep["ok"], (names[i], workspace != 0, rep)


def test_split_k_is_deterministic(capi, ops):
    m, n, k = 64, 1024, 16384
    g = torch.Generator().manual_seed(9)
    a, b = torch.randn(m, k, generator=g).cuda(), torch.randn(k, n, generator=g).cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, None, d, 1.0, 0.0, ops)
    assert plan.name(0).endswith(("_SplitK", "_DeepK")), plan.names()
    # Every MFMA split-k Primitive reduces its partial tiles in a fixed order;
    # the deep-k kernel's last-arriving workgroup too, whichever one it is
    # (more runs: the arrival order changes from run to run).
    s = torch.cuda.current_stream().cuda_stream
    split = [i for i, nm in enumerate(plan.names()) if nm.endswith(("_SplitK", "_DeepK")) and "Mfma" in nm]
    assert len(split) >= 4 and any(plan.name(i).endswith("_DeepK") for i in split), plan.names()
    for i in split:
        outs = []
        for _ in range(12 if plan.name(i).endswith("_DeepK") else 3):
            plan.execute(i, s)
            torch.cuda.synchronize()
            outs.append(d.clone())
        assert all(torch.equal(outs[0], o) for o in outs[1:]), plan.name(i)


def test_skinny_gemv_is_deterministic(capi, ops, oracle):
    # The m <= 8 streaming Primitives also reduce their k splits in a fixed
    # order (partial slices, then the split-k reduction): repeated runs agree
    # bit for bit and match fp64 to the usual bar.
    m, n, k = 4, 4096, 8192
    g = torch.Generator().manual_seed(11)
    a, b, c = (torch.randn(m, k, generator=g).cuda(), torch.randn(k, n, generator=g).cuda(),
               torch.randn(m, n, generator=g).cuda())
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, c, d, 1.5, -0.5, ops)
    gemv = [i for i, nm in enumerate(plan.names()) if nm.startswith("Fp32Gemv")]
    assert gemv and plan.name(0).startswith("Fp32Gemv"), plan.names()
    ref = oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), c.cpu().numpy(), 1.5, -0.5)
    s = torch.cuda.current_stream().cuda_stream
    for i in gemv:
        outs = []
        for _ in range(3):
            d.fill_(float("nan"))
            plan.execute(i, s)
            torch.cuda.synchronize()
            outs.append(d.clone())
        assert all(torch.equal(outs[0], o) for o in outs[1:]), plan.name(i)
        rep = oracle.tolerance_check(outs[0].cpu().numpy(), ref, k)
        assert rep["ok"], (plan.name(i), rep)


@pytest.mark.parametrize("m,n,k,col_a", [(1, 8192, 8192, False), (3, 100, 1000, False), (5, 36, 4, False),
                                         (8, 4096, 2052, False), (4, 200, 37, True), (8, 68, 1030, True)])
def test_one_pass_gemv(capi, ops, oracle, m, n, k, col_a):
    # Fp32Gemv: 32 output columns per workgroup over all of k, reduced in the
    # workgroup in a fixed order and written straight to d.  Every row count
    # bucket (1, 2, 4, 8), column counts that leave a partial workgroup, k
    # tails of a column-major a, and repeated runs bit for bit.
    g = torch.Generator().manual_seed(100 + m + k)
    a = torch.randn(k, m, generator=g).t() if col_a else torch.randn(m, k, generator=g)
    b, c = torch.randn(k, n, generator=g), torch.randn(m, n, generator=g)
    a, b, c = a.cuda(), b.cuda(), c.cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, c, d, 1.5, -0.5, ops)
    names = plan.names()
    assert "Fp32Gemv" in names, names
    i = names.index("Fp32Gemv")
    if (m, n, k) == (1, 8192, 8192):
        assert i == 0, names
    ref = oracle.gemm_f64(a.cpu().numpy(), b.cpu().numpy(), c.cpu().numpy(), 1.5, -0.5)
    s = torch.cuda.current_stream().cuda_stream
    outs = []
    for _ in range(3):
        d.fill_(float("nan"))
        plan.execute(i, s)
        torch.cuda.synchronize()
        outs.append(d.clone())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    rep = oracle.tolerance_check(outs[0].cpu().numpy(), ref, k)
    assert rep["ok"], rep


@pytest.mark.parametrize("m,n,k,with_c", [
    (64, 4096, 4096, False),    # BASELINE 5a shape: 4 splits reduced in the launch
    (4096, 64, 4096, True),     # 5b shape, with c
    (100, 200, 4100, True),     # m, n edge tiles, a k tail of 4 (k % 32 != 0)
    (8, 36, 12, False),         # one tile, a k tail only (no whole slice)
    (130, 260, 16388, False),   # many splits, every edge
    (256, 256, 65536, True),    # BASELINE 5c shape with c
])
def test_deep_k_kernel(capi, ops, oracle, m, n, k, with_c):
    """Fp32Mfma16Gemm_64x64_DeepK on edges and tails, with its partials in the
    Plan's own buffer and in a caller workspace full of garbage (the arrival
    counters are cleared before the launch); repeated runs are bit-identical
    whichever workgroup of a tile arrives last."""
    g = torch.Generator().manual_seed(m + n + k)
    a_h, b_h = torch.randn(m, k, generator=g), torch.randn(k, n, generator=g)
    c_h = torch.randn(m, n, generator=g) if with_c else None
    alpha, beta = 0.75, (-1.5 if with_c else 0.0)
    ref = oracle.gemm_f64(a_h, b_h, c_h, alpha, beta)
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a_h.cuda(), b_h.cuda(), None if c_h is None else c_h.cuda(), d, alpha, beta, ops)
    names = plan.names()
    i = names.index("Fp32Mfma16Gemm_64x64_DeepK")
    s = torch.cuda.current_stream().cuda_stream
    need = plan.workspace_bytes(i)
    ws = torch.full((max(need, 16) // 4 + 64,), -1, dtype=torch.int32, device="cuda")  # counters read 0xffffffff
    outs = []
    for run in range(6):
        d.fill_(float("nan"))
        if need and run % 2:
            plan.execute(i, s, ws.data_ptr(), ws.numel() * 4)
        else:
            plan.execute(i, s)
        torch.cuda.synchronize()
        outs.append(d.clone())
    rep = oracle.tolerance_check(outs[0].cpu().numpy(), ref, k)
    assert rep["ok"], (names[i], need, rep)
    assert rep["max_abs_err"] <= 1e-2 * rep["bound"], rep  # far inside the bar, not just under it
    assert all(torch.equal(outs[0], o) for o in outs[1:]), names[i]


@pytest.mark.parametrize("m,n,k,with_c,pad", [
    (256, 256, 32, False, 0),     # one stage
    (512, 256, 96, True, 4),      # an odd stage count (the pipeline's tail copy), padded rows
    (256, 512, 1024, True, 0),    # a long even run
    (768, 1024, 2080, False, 8),  # 12 tiles, 65 stages
    (300, 200, 64, True, 4),      # edge tiles in m and n (clamped loads, dropped stores)
    (40, 24, 32, False, 0),       # smaller than one tile
])
def test_fp32_dma_tile(capi, ops, oracle, m, n, k, with_c, pad):
    """Fp32Mfma16Gemm_256x256_Dma (operands staged into LDS by DMA): one, odd and long stage
    counts, edge tiles, row strides padded past the used extent with NaN (a read out of a row
    fails the check), d inside a 7.0-filled store (nothing written outside it), twice in a row
    bit for bit."""
    g = torch.Generator().manual_seed(m + n + k)
    a_h, b_h = torch.randn(m, k, generator=g), torch.randn(k, n, generator=g)
    c_h = torch.randn(m, n, generator=g) if with_c else None
    alpha, beta = 1.25, (0.5 if with_c else 0.0)
    ref = oracle.gemm_f64(a_h, b_h, c_h, alpha, beta)
    a_s = torch.full((m, k + pad), float("nan")); a_s[:, :k] = a_h
    b_s = torch.full((k, n + pad), float("nan")); b_s[:, :n] = b_h
    a_d, b_d = a_s.cuda()[:, :k], b_s.cuda()[:, :n]
    d_s = torch.full((m + 1, n + pad), 7.0, device="cuda")
    d = d_s[:m, :n]
    plan = capi.plan_for(a_d, b_d, None if c_h is None else c_h.cuda(), d, alpha, beta, ops)
    names = plan.names()
    i = names.index("Fp32Mfma16Gemm_256x256_Dma")
    keep = torch.ones_like(d_s, dtype=torch.bool)
    keep[:m, :n] = False
    outs = []
    for _ in range(2):
        d.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append(d.clone())
        assert torch.all(d_s[keep] == 7.0), "wrote outside d"
    rep = oracle.tolerance_check(outs[0].cpu().numpy(), ref, k)
    assert rep["ok"], (names[i], rep)
    assert rep["max_abs_err"] <= 1e-2 * rep["bound"], rep
    assert torch.equal(outs[0], outs[1])


def test_fp32_dma_tile_layouts_and_k_tails(capi, ops):
    a = torch.zeros(256, 64, device="cuda")
    b = torch.zeros(64, 256, device="cuda")
    d = torch.empty(256, 256, device="cuda")
    assert "Fp32Mfma16Gemm_256x256_Dma" in capi.plan_for(a, b, None, d, 1.0, 0.0, ops).names()
    # column-major b: the row-major kernel does not apply; a k tail (k % 32 != 0) it stages itself
    assert "Fp32Mfma16Gemm_256x256_Dma" not in capi.plan_for(a, b.t().contiguous().t(), None, d, 1.0, 0.0, ops).names()
    a3 = torch.zeros(256, 48, device="cuda")
    assert "Fp32Mfma16Gemm_256x256_Dma" in capi.plan_for(a3, b[:48], None, d, 1.0, 0.0, ops).names()
    # the 128x128 tile takes a column-major b, a column-major a, or both; the 64x128 split tile
    # (wave rows of 32) takes no column-major a
    a, b = torch.zeros(256, 1024, device="cuda"), torch.zeros(1024, 256, device="cuda")  # deep enough to split
    for at, bt in ((False, False), (False, True), (True, False), (True, True)):
        names = capi.plan_for(a.t().contiguous().t() if at else a, b.t().contiguous().t() if bt else b, None, d,
                              1.0, 0.0, ops).names()
        assert "Fp32Mfma16Gemm_128x128_Dma" in names, (at, bt, names)
        assert ("Fp32Mfma16Gemm_64x128_Dma_SplitK" in names) == (not at), (at, bt, names)


@pytest.mark.parametrize("m,n,k,with_c,splits", [
    (64, 4096, 4096, False, 16),   # BASELINE 5a shape at its split count
    (4096, 64, 4096, True, 16),    # 5b, with c
    (64, 1024, 4096, False, 64),
    (100, 1000, 2080, True, 5),    # edge tiles in m and n, an odd split count
    (300, 200, 1024, False, 3),
    (64, 256, 512, True, 2),
    (256, 512, 4128, False, 16),   # 15 used splits of 16 asked (chunk rounding)
    (70, 2052, 3200, True, 7),
    (1024, 4096, 512, False, 2),   # many tiles per CU: the epilogue's store-data hazard showed here
    (4096, 1024, 512, True, 2),
])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)],
                         ids=["nn", "nt", "tn", "tt"])
def test_fp32_split_k_at_forced_split_counts(capi, oracle, m, n, k, with_c, splits, ta, tb):
    """Every DMA split-k tile (partial tiles, then the reduction kernel) in every operand
    orientation it has, and the deep-k kernel
    (reduction in the launch by the tile's last workgroup) at split counts forced through the
    test hook rather than picked by the cost model: against fp64, d inside a 7.0-filled store,
    bit-identical over repeats with the partials in the Plan's buffer or in a caller workspace
    full of garbage, then again at 2 splits and back on the same buffers."""
    if ta and m % 4:
        pytest.skip("a column-major a needs m % 4 == 0 for the 128-bit kernels")
    t = capi.testing_lib()
    ops = capi.GemmOps(l=t, order=("d", "beta", "alpha", "c", "b", "a"))
    g = torch.Generator().manual_seed(m * 7 + n + k + splits)
    a_h, b_h = torch.randn(m, k, generator=g), torch.randn(k, n, generator=g)
    c_h = torch.randn(m, n, generator=g) if with_c else None
    alpha, beta = 0.75, (1.5 if with_c else 0.0)
    ref = oracle.gemm_f64(a_h, b_h, c_h, alpha, beta)
    a_d = a_h.t().contiguous().cuda().t() if ta else a_h.cuda()
    b_d = b_h.t().contiguous().cuda().t() if tb else b_h.cuda()
    c_d = None if c_h is None else c_h.cuda()
    d_s = torch.full((m + 1, n + 4), 7.0, device="cuda")
    d = d_s[:m, :n]
    keep = torch.ones_like(d_s, dtype=torch.bool)
    keep[:m, :n] = False
    # Column-major a: the tiles with wave rows in runs of 64; column-major b: all but 256x256; the
    # deep-k kernel takes row-major a and b only.
    tiles = ("128x128", "64x256", "256x64") + (() if ta else ("64x128", "128x64", "64x64"))
    tiles += () if ta or tb else ("256x256",)
    names = [f"Fp32Mfma16Gemm_{tl}_Dma_SplitK" for tl in tiles] + ([] if ta or tb else ["Fp32Mfma16Gemm_64x64_DeepK"])
    s = torch.cuda.current_stream().cuda_stream
    try:
        for s_now in (splits, 2, splits):
            t.ftrainTestingForceSplits(s_now)
            plan = capi.plan_for(a_d, b_d, c_d, d, alpha, beta, ops)
            for name in names:
                assert name in plan.names(), (name, plan.names())
                i = plan.names().index(name)
                need = plan.workspace_bytes(i)
                ws = torch.full((max(need, 16) // 4 + 64,), -1, dtype=torch.int32, device="cuda")
                outs = []
                for run in range(3):
                    d.fill_(float("nan"))
                    if need or run == 2:  # a caller workspace full of garbage (counters cleared first)
                        plan.execute(i, s, ws.data_ptr(), ws.numel() * 4)
                    else:
                        plan.execute(i, s)
                    torch.cuda.synchronize()
                    outs.append(d.clone())
                    assert torch.all(d_s[keep] == 7.0), (name, "wrote outside d")
                rep = oracle.tolerance_check(outs[0].cpu().numpy(), ref, k)
                assert rep["ok"], (name, s_now, rep)
                assert rep["max_abs_err"] <= 1e-2 * rep["bound"], (name, s_now, rep)
                assert all(torch.equal(outs[0], o) for o in outs[1:]), (name, s_now)
            plan.close()
    finally:
        t.ftrainTestingForceSplits(0)


@pytest.mark.parametrize("m,n,k,ta,tb", [(2048, 2048, 512, False, False), (4096, 1024, 256, False, False),
                                          (2048, 2048, 512, False, True), (1000, 1500, 544, False, True),
                                          (2048, 2048, 512, True, False), (1000, 1500, 544, True, False),
                                          (1500, 1000, 544, True, True)])
def test_fp32_dma_whole_k_tiles_every_output(capi, ops, oracle, m, n, k, ta, tb):
    """The whole-k DMA tiles over many rounds of workgroups, every output checked, five runs:
    a store whose data registers were overwritten right after it (a hardware hazard the
    compiler does not cover for buffer stores) showed only under such load, as a few stray
    dwords per launch.  ta / tb: a / b column-major (storage k x m / n x k), on the tiles that
    take them (1000 x 1500 has edge tiles in m and n)."""
    g = torch.Generator().manual_seed(m + n + k)
    a_h, b_h, c_h = torch.randn(m, k, generator=g), torch.randn(k, n, generator=g), torch.randn(m, n, generator=g)
    ref = oracle.gemm_f64(a_h, b_h, c_h, 1.0, 0.5)
    d = torch.empty(m, n, device="cuda")
    a_d = a_h.t().contiguous().cuda().t() if ta else a_h.cuda()
    b_d = b_h.t().contiguous().cuda().t() if tb else b_h.cuda()
    plan = capi.plan_for(a_d, b_d, c_h.cuda(), d, 1.0, 0.5, ops)
    s = torch.cuda.current_stream().cuda_stream
    tiles = ("128x128",) if ta else ("128x128", "64x128", "128x64") if tb else ("256x256", "128x128", "64x128", "128x64")
    for name in (f"Fp32Mfma16Gemm_{t}_Dma" for t in tiles):
        i = plan.names().index(name)
        for _ in range(5):
            d.fill_(float("nan"))
            plan.execute(i, s)
            torch.cuda.synchronize()
            rep = oracle.tolerance_check(d.cpu().numpy(), ref, k)
            assert rep["ok"] and rep["max_abs_err"] <= 1e-2 * rep["bound"], (name, rep)
