"""Operands beyond 4 GiB (64-bit addressing), called through the C ABI.

Every kernel forms its addresses from 64-bit matrix bases plus row offsets
(`(size_t)row * ld`); the DMA tiles build per-tile 64-bit bases and keep
32-bit offsets inside a tile.  These cases put rows of a (or rows of b, for
the skinny kernels) past byte 2^32 and run every Primitive of the Plan, each
checked on sampled rows or columns -- the last ones included -- against the
fp64 oracle.  The reference's overflow rule (`problem.cpp:13-56`) admits
these sizes, so every Primitive must get them right.
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


def device_randn(shape, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(*shape, generator=g, device="cuda")


def run_every_primitive(capi, plan, d, check, label):
    names = plan.names()
    ws = None
    for i, name in enumerate(names):
        print(f"[large] {label} primitive {i} {name}", flush=True)
        need = plan.workspace_bytes(i)
        if need and (ws is None or ws.numel() < need):
            ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        d.fill_(float("nan"))
        s = torch.cuda.current_stream().cuda_stream
        plan.execute(i, s, *((ws.data_ptr(), ws.numel()) if need else (0, 0)))
        torch.cuda.synchronize()
        check(name)
    return names


def test_a_beyond_4_gib(capi, oracle):
    m, n, k = 139264, 256, 8192  # a: 4.25 GiB; rows from 131072 on start past byte 2^32
    assert m * k * 4 > (1 << 32)
    a = device_randn((m, k), 1)
    b = device_randn((k, n), 2)
    d = torch.empty(m, n, device="cuda")
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 48).astype(np.int64),
                                     np.arange(131070, 131074), np.arange(m - 12, m)]))
    idx = torch.from_numpy(rows).cuda()
    a_rows = a.index_select(0, idx).cpu().numpy()
    b_h = b.cpu().numpy()
    ref = oracle.gemm_f64(a_rows, b_h, None, 1.0, 0.0)

    def check(name):
        got = d.index_select(0, idx).cpu().numpy()
        rep = oracle.tolerance_check(got, ref, k)
        assert rep["ok"], (name, rep)

    plan = capi.plan_for(a, b, None, d, 1.0, 0.0)
    names = run_every_primitive(capi, plan, d, check, f"{m}x{n}x{k}")
    assert any("_Dma" in nm for nm in names), names
    del a, b, d


def test_gemv_b_beyond_4_gib(capi, oracle):
    m, n, k = 1, 8192, 139264  # b: 4.25 GiB; its rows from 131072 on start past byte 2^32
    assert k * n * 4 > (1 << 32)
    a = device_randn((m, k), 3)
    b = device_randn((k, n), 4)
    c = device_randn((m, n), 5)
    d = torch.empty(m, n, device="cuda")
    cols = np.unique(np.concatenate([np.linspace(0, n - 1, 40).astype(np.int64), np.arange(n - 8, n)]))
    cidx = torch.from_numpy(cols).cuda()
    b_cols = b.index_select(1, cidx).cpu().numpy()
    ref = oracle.gemm_f64(a.cpu().numpy(), b_cols, c.index_select(1, cidx).cpu().numpy(), 0.5, 2.0)

    def check(name):
        got = d.index_select(1, cidx).cpu().numpy()
        rep = oracle.tolerance_check(got, ref, k)
        assert rep["ok"], (name, rep)

    plan = capi.plan_for(a, b, c, d, 0.5, 2.0)
    names = run_every_primitive(capi, plan, d, check, f"{m}x{n}x{k}")
    assert "Fp32Gemv" in names, names
    del a, b, c, d
