"""GPU parity of strided and transposed operands, called through the C ABI.

The reference accepts row-major contiguous matrices only
(src/primitive/hygon/gemm/fp32_gemm.cpp:39-46); this build also accepts
explicit strides with one unit dimension: a and b row- or column-major, c and
d in one shared orientation, each with its own leading dimension.  Every
Primitive of each Plan is compared with the fp64 oracle on the logical
matrices, to the north-star bar max|d - ref| <= 1e-4 * sqrt(k) * max|ref|.

The storage around each view is filled with NaN, so a kernel that reads
outside its operand (a wrong leading dimension or orientation) fails the
comparison, and the padding of d is checked to stay untouched.
"""

import itertools

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


@pytest.fixture(scope="module")
def ops(capi):
    return capi.GemmOps()


def placed(x: np.ndarray, col_major: bool, pad: int, fill: float = float("nan")):
    """Device view holding the values of x (rows x cols) in the requested
    orientation, with `pad` extra elements per leading dimension, inside a
    storage filled with `fill`.  Returns (view tensor, storage tensor)."""
    r, c = x.shape
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    if col_major:
        store = torch.full((c, r + pad), fill, dtype=torch.float32)
        store[:, :r] = t.t()
        store = store.cuda()
        return store[:, :r].t(), store
    store = torch.full((r, c + pad), fill, dtype=torch.float32)
    store[:, :c] = t
    store = store.cuda()
    return store[:, :c], store


def view(capi, t):
    """Continuous index type for a contiguous tensor, explicit strides otherwise."""
    if t.is_contiguous():
        return capi.matrix(t)
    return capi.View(t.data_ptr(), list(t.shape), index_type=capi.INDEX_INVALID, strides=list(t.stride()))


def run_every_primitive(capi, ops, oracle, m, n, k, la, lb, lcd, pad, with_c, alpha=1.25, beta=-0.5, seed=0):
    g = np.random.default_rng(seed)
    a = g.standard_normal((m, k)).astype(np.float32)
    b = g.standard_normal((k, n)).astype(np.float32)
    c = g.standard_normal((m, n)).astype(np.float32) if with_c else None
    ref = oracle.gemm_f64(a, b, c, alpha, beta)
    av, _ = placed(a, la, pad)
    bv, _ = placed(b, lb, pad)
    cv = placed(c, lcd, pad)[0] if with_c else None
    sentinel = 12345.0
    dv, dstore = placed(np.zeros((m, n), np.float32), lcd, pad, fill=sentinel)
    al, be = capi.HostScalar(alpha), capi.HostScalar(beta)
    cview = view(capi, cv) if with_c else capi.View(None, [m, n])
    args = ops.args(view(capi, av), view(capi, bv), cview, view(capi, dv), al.view, be.view)
    plan = args.plan()
    args.close()
    names = plan.names()
    pad_mask = torch.ones_like(dstore, dtype=torch.bool)
    if lcd:
        pad_mask[:, :m] = False
    else:
        pad_mask[:, :n] = False
    for i, name in enumerate(names):
        dv.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        rep = oracle.tolerance_check(dv.cpu().numpy(), ref, k)
        assert rep["ok"], (name, m, n, k, la, lb, lcd, pad, rep)
        assert torch.all(dstore[pad_mask] == sentinel), (name, "wrote outside d")
    return names


LAYOUTS = list(itertools.product((False, True), (False, True), (False, True)))


@pytest.mark.parametrize("la,lb", list(itertools.product((False, True), (False, True))))
@pytest.mark.parametrize("m,n,k,pad", [(256, 256, 20, 4), (256, 256, 44, 0), (384, 256, 1000, 4), (512, 512, 4100, 0),
                                       (64, 4096, 4100, 0), (4096, 64, 4100, 0), (256, 256, 65540, 0)])
def test_fp32_dma_tiles_with_a_k_tail(capi, ops, oracle, la, lb, m, n, k, pad):
    # k not a multiple of 32: the fp32 DMA tiles run the whole stages through their pipeline and stage
    # the partial last one by ordinary loads, zeros past k (less than one stage; one stage and 12 more;
    # 31 stages and 8 more; deep k and skinny shapes on the split tiles, whose last split holds the
    # tail).  Every Primitive of each Plan, every operand orientation, NaN past each leading dimension.
    names = run_every_primitive(capi, ops, oracle, m, n, k, la, lb, False, pad, with_c=True, seed=k)
    assert any("_Dma" in nm for nm in names), names


@pytest.mark.parametrize("k", [2, 3, 5, 31, 33, 63, 97, 1001])
def test_fp32_dma_tiles_any_k_with_column_major_a(capi, ops, oracle, k):
    # A column-major a and a row-major b are both read along k rows, so k need not be a multiple of
    # the 4-element load: the fp32 DMA tiles' partial last stage is staged row by row, zeros past k.
    names = run_every_primitive(capi, ops, oracle, 132, 260, k, True, False, False, 4, with_c=True, seed=k)
    assert any("_Dma" in nm for nm in names), names


@pytest.mark.parametrize("la,lb,lcd", LAYOUTS)
@pytest.mark.parametrize("m,n,k,pad", [(256, 192, 160, 4), (256, 192, 150, 4), (129, 67, 37, 3), (64, 64, 1024, 0)])
def test_layouts_every_primitive(capi, ops, oracle, la, lb, lcd, m, n, k, pad):
    if pad == 0 and not (la or lb or lcd):
        pytest.skip("plain continuous layout is covered by test_gpu_gemm.py")
    names = run_every_primitive(capi, ops, oracle, m, n, k, la, lb, lcd, pad, with_c=True)
    assert "Fp32Gemm" in names


def test_column_major_d_without_c(capi, ops, oracle):
    run_every_primitive(capi, ops, oracle, 96, 160, 64, False, True, True, 4, with_c=False)


def test_transposed_skinny_rows_use_split_k(capi, ops, oracle):
    # m = 4 rows of a column-major a, deep k: the skinny kernel and split-k tiles.
    names = run_every_primitive(capi, ops, oracle, 4, 512, 4096, True, False, False, 4, with_c=True)
    assert any(n.startswith("Fp32Gemv") for n in names), names


def test_transposed_headline_shape_sampled(capi, ops, oracle):
    # a^T b at 2048^3 (the dgrad orientation) on Primitive 0, checked on sampled rows.
    m = n = k = 2048
    gen = torch.Generator().manual_seed(2026)
    a = torch.randn(m, k, generator=gen)
    b = torch.randn(k, n, generator=gen)
    at = a.t().contiguous().cuda()  # storage k x m; a = at.t()
    bd = b.cuda()
    d = torch.empty(m, n, device="cuda")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    av = at.t()
    args = ops.args(view(capi, av), view(capi, bd), capi.View(None, [m, n]), capi.matrix(d), al.view, be.view)
    plan = args.plan()
    args.close()
    assert plan.name(0).startswith("Fp32Mfma"), plan.names()
    plan.execute(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    rows = np.random.default_rng(1).choice(m, 64, replace=False)
    ref = oracle.sampled_rows_f64(a, b, None, 1.0, 0.0, rows)
    rep = oracle.tolerance_check(d.cpu().numpy()[rows], ref, k)
    assert rep["ok"], rep
