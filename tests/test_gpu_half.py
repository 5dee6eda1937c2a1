"""GPU parity of the bf16 / fp16 GEMM variants, called through the C ABI.

a and b in bf16 or fp16, fp32 accumulation, c and d in fp32 or the input
type.  The reference names both element types in its numeric-type enum
(include/flash_train/common.h:38-65) but ships only the fp32 kernel
(src/primitive/hygon/gemm/fp32_gemm.hip:18-31), whose formula these variants
follow.  Each result is compared with the fp64 oracle of the exactly decoded
inputs (oracle.gemm_f64_typed) under the north-star bar
max|d - ref| <= 1e-4 * sqrt(k) * max|ref|, widened for a bf16 / fp16 d by
that type's rounding: |d - ref| <= bound * (1 + u) + u * |ref|,
u = 2^-8 (bf16) or 2^-11 (fp16).  Operand storage is padded with NaN so an
out-of-bounds read fails the comparison.
"""

import itertools

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


@pytest.fixture(scope="module")
def capi():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible device")
    from flash_train import capi as c

    return c


@pytest.fixture(scope="module")
def ops(capi):
    return capi.GemmOps()


def placed(x: np.ndarray, dtype, col_major: bool, pad: int, fill=float("nan")):
    """Device tensor view with the values of x (already representable in dtype), row- or
    column-major with `pad` spare elements per leading dimension, in a storage filled with `fill`."""
    r, c = x.shape
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dtype)
    if col_major:
        store = torch.full((c, r + pad), fill, dtype=dtype)
        store[:, :r] = t.t()
        store = store.cuda()
        return store[:, :r].t(), store
    store = torch.full((r, c + pad), fill, dtype=dtype)
    store[:, :c] = t
    store = store.cuda()
    return store[:, :c], store


def rounded(x: np.ndarray, kind: str) -> np.ndarray:
    """x rounded to the 16-bit type and back to fp32 values."""
    return torch.from_numpy(x).to(DT[kind]).float().numpy()


def run_case(capi, ops, oracle, kind, cd, m, n, k, la, lb, lcd=False, pad=0, with_c=True, alpha=1.5, beta=-0.75,
             seed=0, every=True):
    g = np.random.default_rng(seed)
    a = rounded(g.standard_normal((m, k)).astype(np.float32), kind)
    b = rounded(g.standard_normal((k, n)).astype(np.float32), kind)
    c = g.standard_normal((m, n)).astype(np.float32) if with_c else None
    if c is not None and cd != "fp32":
        c = rounded(c, cd)
    ref = oracle.gemm_f64(a, b, c, alpha, beta)
    av, _ = placed(a, DT[kind], la, pad)
    bv, _ = placed(b, DT[kind], lb, pad)
    cv = placed(c, DT[cd], lcd, pad)[0] if with_c else None
    dv, dstore = placed(np.zeros((m, n), np.float32), DT[cd], lcd, pad, fill=7.0)
    al, be = capi.HostScalar(alpha), capi.HostScalar(beta)
    cview = capi.matrix(cv) if with_c else capi.View(None, [m, n], numeric_type=capi.TORCH_NUMERIC_TYPES[DT[cd]])
    args = ops.args(capi.matrix(av), capi.matrix(bv), cview, capi.matrix(dv), al.view, be.view)
    plan = args.plan()
    args.close()
    names = plan.names()
    assert all(nm.startswith(kind.capitalize()) for nm in names), names
    keep = torch.ones_like(dstore, dtype=torch.bool)
    if lcd:
        keep[:, :m] = False
    else:
        keep[:, :n] = False
    for i, name in enumerate(names if every else names[:1]):
        dv.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        rep = oracle.tolerance_check(dv.float().cpu().numpy(), ref, k, cd)
        assert rep["ok"], (name, kind, cd, m, n, k, la, lb, lcd, pad, rep)
        assert torch.all(dstore[keep].float() == 7.0), (name, "wrote outside d")
    return names


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("cd", ["fp32", "same"])
@pytest.mark.parametrize("la,lb", list(itertools.product((False, True), (False, True))))
@pytest.mark.parametrize("m,n,k,pad", [(256, 192, 160, 8), (129, 67, 37, 3), (384, 256, 1024, 0),
                                       (384, 200, 1024, 8)])  # last: n-edge tiles with no k tail (clamped columns)
def test_half_every_primitive(capi, ops, oracle, kind, cd, la, lb, m, n, k, pad):
    run_case(capi, ops, oracle, kind, kind if cd == "same" else "fp32", m, n, k, la, lb, pad=pad)


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("cd", ["fp32", "same"])
@pytest.mark.parametrize("la,lb", list(itertools.product((False, True), (False, True))))
@pytest.mark.parametrize("m,n,k,pad,with_c", [(256, 256, 64, 8, True), (512, 256, 192, 8, False),
                                              (256, 512, 1024, 0, True), (296, 520, 128, 8, True),
                                              (40, 24, 64, 0, False)])
def test_half_dma_tile(capi, ops, oracle, kind, cd, la, lb, m, n, k, pad, with_c):
    # The 256x256 and 128x128 tiles with LDS staging by DMA (the 128x128 one also split-k): one
    # stage (k = 64), an odd stage count (the tail
    # copy of the pipeline), a long even one, edge tiles in m and n (loads clamped, stores
    # checked) and a matrix smaller than one tile; every operand orientation, NaN past each
    # leading dimension's used extent, 7.0 around d (nothing written outside it).
    names = run_case(capi, ops, oracle, kind, kind if cd == "same" else "fp32", m, n, k, la, lb, pad=pad,
                     with_c=with_c, seed=k + pad)
    assert f"{kind.capitalize()}MfmaGemm_256x256_Dma" in names, names
    assert f"{kind.capitalize()}MfmaGemm_128x128_Dma" in names, names
    if k >= 512:
        assert f"{kind.capitalize()}MfmaGemm_128x128_Dma_SplitK" in names, names


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("cd", ["fp32", "same"])
@pytest.mark.parametrize("la,lb", list(itertools.product((False, True), (False, True))))
@pytest.mark.parametrize("m,n,k,pad,with_c", [(256, 256, 72, 8, True), (296, 520, 40, 0, True),
                                              (384, 256, 1000, 8, False), (64, 1024, 8200, 0, True),
                                              (384, 4096, 4104, 0, False)])
def test_half_dma_tiles_with_a_k_tail(capi, ops, oracle, kind, cd, la, lb, m, n, k, pad, with_c):
    # k not a multiple of 64: the DMA tiles run the whole stages through their pipeline and stage the
    # partial last one by ordinary loads, zeros past k (one stage and 8 more k; less than one stage;
    # 15 stages and 40 more; deep k on the split tiles, whose last split holds the tail).  Every
    # Primitive of each Plan, every operand orientation, NaN past each leading dimension.
    names = run_case(capi, ops, oracle, kind, kind if cd == "same" else "fp32", m, n, k, la, lb, pad=pad,
                     with_c=with_c, seed=k + m)
    assert any("_Dma" in nm for nm in names), names


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("k", [2, 7, 9, 63, 65, 101, 127, 129, 1001])
def test_half_dma_tiles_any_k_with_column_major_a(capi, ops, oracle, kind, k):
    # A column-major a and a row-major b are both read along k rows, so k need not be a multiple of
    # the 8-element load: the DMA tiles' partial last stage is staged row by row, zeros past k, and
    # a k below one stage runs the pipeline on a dummy buffer.  Every Primitive of the Plan.
    names = run_case(capi, ops, oracle, kind, "fp32", 136, 264, k, True, False, pad=8, with_c=True, seed=k)
    assert any("_Dma" in nm for nm in names), names


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("cd", ["fp32", "same"])
@pytest.mark.parametrize("la,lb", list(itertools.product((False, True), (False, True))))
@pytest.mark.parametrize("m,n,k,pad,with_c", [(64, 4096, 4096, 0, False), (40, 200, 1024, 8, True),
                                              (1, 136, 576, 8, True), (64, 1024, 8192, 0, True)])
def test_half_dma_64_row_split_tile(capi, ops, oracle, kind, cd, la, lb, m, n, k, pad, with_c):
    # The 64x128 split-k DMA tile (m of at most 64, row-major a): a full-height tile, partial ones
    # (rows clamped, stores dropped), an n edge, uneven splits (576 = 320 + 256) and deep k; every
    # Primitive of each Plan.  A column-major a leaves it out of the Plan.
    names = run_case(capi, ops, oracle, kind, kind if cd == "same" else "fp32", m, n, k, la, lb, pad=pad,
                     with_c=with_c, seed=m + k + pad)
    tile = f"{kind.capitalize()}MfmaGemm_64x128_Dma_SplitK"
    assert (tile in names) == (not la), names


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("tb", [False, True], ids=["b_row", "b_col"])
@pytest.mark.parametrize("k,splits", [(256, 4), (512, 4), (768, 4), (1024, 4), (1280, 4), (1800, 4), (264, 4),
                                      (200, 2), (4096, 8)])
def test_half_64_row_split_tile_at_forced_split_counts(capi, oracle, kind, tb, k, splits):
    """The 64x128 split tile runs a ring of three stage buffers.  Split counts forced through the test
    hook give split ranges of 1, 2, 3, 4, 5 and 8 whole stages (every way out of the ring's
    three-stage loop) and, with a k tail, a last split of 4 stages + 8 k, 1 stage + 8 k or only 8 k
    (264 = 128 + 128 + 8).  Against fp64, d inside a 7.0-filled store, bit-identical over repeats."""
    t = capi.testing_lib()
    ops = capi.GemmOps(l=t)
    m, n = 64, 392
    g = np.random.default_rng(k * 3 + splits)
    a = rounded(g.standard_normal((m, k)).astype(np.float32), kind)
    b = rounded(g.standard_normal((k, n)).astype(np.float32), kind)
    c = g.standard_normal((m, n)).astype(np.float32)
    ref = oracle.gemm_f64(a, b, c, 0.5, -1.25)
    av, _ = placed(a, DT[kind], False, 8)
    bv, _ = placed(b, DT[kind], tb, 8)
    cv, _ = placed(c, torch.float32, False, 4)
    dv, dstore = placed(np.zeros((m, n), np.float32), torch.float32, False, 4, fill=7.0)
    keep = torch.ones_like(dstore, dtype=torch.bool)
    keep[:, :n] = False
    name = f"{kind.capitalize()}MfmaGemm_64x128_Dma_SplitK"
    try:
        t.ftrainTestingForceSplits(splits)
        plan = capi.plan_for(av, bv, cv, dv, 0.5, -1.25, ops)
        assert name in plan.names(), plan.names()
        i = plan.names().index(name)
        outs = []
        for _ in range(3):
            dv.fill_(float("nan"))
            plan.execute(i, torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            outs.append(dv.clone())
            assert torch.all(dstore[keep] == 7.0), "wrote outside d"
        rep = oracle.tolerance_check(outs[0].cpu().numpy(), ref, k)
        assert rep["ok"], (kind, tb, k, splits, rep)
        assert all(torch.equal(outs[0], o) for o in outs[1:])
        plan.close()
    finally:
        t.ftrainTestingForceSplits(0)


@pytest.mark.parametrize("cd", ["fp32", "same"])
def test_half_split_k_wide_reduction(capi, ops, oracle, cd):
    # 384x4096 outputs at k = 4096: the split-k tile's reduction runs one thread per output unit
    # (four fp32 values with fp32 c and d, one with a bf16 d); every Primitive of the Plan.
    names = run_case(capi, ops, oracle, "bf16", "bf16" if cd == "same" else "fp32", 384, 4096, 4096, False, False,
                     seed=9)
    assert "Bf16MfmaGemm_128x128_SplitK" in names, names


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_half_dma_tile_exact_and_repeatable(capi, ops, kind):
    # Integer inputs in [-8, 8] (exact in fp32 for this k): the DMA tile equals the integer
    # product bit for bit, on a run after another shape (so the LDS held other data) and twice.
    g = np.random.default_rng(5)
    m, n, k = 512, 256, 320
    a = g.integers(-8, 9, (m, k)).astype(np.float32)
    b = g.integers(-8, 9, (k, n)).astype(np.float32)
    exact = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    at = torch.from_numpy(a).to(DT[kind]).cuda()
    bt = torch.from_numpy(b).to(DT[kind]).cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(at, bt, None, d, 1.0, 0.0, ops)
    for tile in ("256x256", "128x128"):
        i = plan.names().index(f"{kind.capitalize()}MfmaGemm_{tile}_Dma")
        for _ in range(2):
            d.fill_(float("nan"))
            plan.execute(i, torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(d.cpu().numpy(), exact)


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("lb", [False, True])
def test_half_dma_tile_prefetching_a_large_b(capi, ops, kind, lb):
    # A b of more than 256 MiB (4096 x 32776, 268 MB) selects the 256x256 DMA tile's form that
    # prefetches b into L2 four stages ahead.  Integer inputs in [-2, 2] make the fp32 result exact:
    # it must equal the fp64 product bit for bit, with an edge tile in m and a last column tile of 8
    # (the prefetched lines clamped onto the matrix), and b row- or column-major with a padded ld.
    m, n, k = 384, 32776, 4096
    gen = torch.Generator(device="cuda").manual_seed(17)
    a = torch.randint(-2, 3, (m, k), device="cuda", generator=gen).to(DT[kind])
    b_int = torch.randint(-2, 3, (k, n), device="cuda", generator=gen)
    if lb:
        store = torch.full((n, k + 8), float("nan"), dtype=DT[kind], device="cuda")
        store[:, :k] = b_int.t().to(DT[kind])
        b = store[:, :k].t()
    else:
        store = torch.full((k, n + 8), float("nan"), dtype=DT[kind], device="cuda")
        store[:, :n] = b_int.to(DT[kind])
        b = store[:, :n]
    exact = (a.double() @ b_int.double()).float()
    del b_int
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(a, b, None, d, 1.0, 0.0, ops)
    i = plan.names().index(f"{kind.capitalize()}MfmaGemm_256x256_Dma")
    for _ in range(2):
        d.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(d, exact), (kind, lb, (d - exact).abs().max().item())


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
@pytest.mark.parametrize("cd", ["fp32", "same"])
@pytest.mark.parametrize("m,n,k,pad", [(1, 8192, 8192, 0), (2, 200, 1000, 8), (1, 64, 8, 0), (2, 4096, 2056, 0),
                                       (3, 64, 64, 0), (4, 128, 1024, 8), (5, 64, 64, 0)])
def test_half_one_pass_gemv(capi, ops, oracle, kind, cd, m, n, k, pad):
    # Bf16Gemv / Fp16Gemv: 64 output columns per workgroup over all of k, written straight to d,
    # for one or two rows of a (three and more go to the tile kernels); partial last workgroups and
    # padded strides.
    names = run_case(capi, ops, oracle, kind, kind if cd == "same" else "fp32", m, n, k, False, False, pad=pad,
                     seed=m + k)
    assert (f"{kind.capitalize()}Gemv" in names) == (m <= 2), names
    if (m, n, k) == (1, 8192, 8192):
        assert names[0] == f"{kind.capitalize()}Gemv", names


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_half_column_major_d_and_no_c(capi, ops, oracle, kind):
    run_case(capi, ops, oracle, kind, "fp32", 96, 160, 64, False, True, lcd=True, pad=8, with_c=False)
    run_case(capi, ops, oracle, kind, kind, 96, 160, 64, True, False, lcd=True, pad=8, with_c=True)


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_half_deep_k_uses_split_k(capi, ops, oracle, kind):
    names = run_case(capi, ops, oracle, kind, "fp32", 128, 128, 16384, False, True)
    assert any("SplitK" in nm for nm in names), names


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_half_exact_on_small_integers(capi, ops, kind):
    # Integer inputs in [-8, 8]: every product and partial sum is exact in fp32 for k <= 2^16 / 64,
    # so an fp32 d must equal the integer product bit for bit on every Primitive.
    g = np.random.default_rng(11)
    m, n, k = 160, 96, 256
    a = g.integers(-8, 9, (m, k)).astype(np.float32)
    b = g.integers(-8, 9, (k, n)).astype(np.float32)
    exact = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    at = torch.from_numpy(a).to(DT[kind]).cuda()
    bt = torch.from_numpy(b).to(DT[kind]).cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(at, bt, None, d, 1.0, 0.0, ops)
    for i in range(len(plan)):
        d.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(d.cpu().numpy(), exact, err_msg=plan.name(i))


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_half_nan_inf_propagation(capi, ops, oracle, kind):
    m, n, k = 64, 64, 64
    g = np.random.default_rng(2)
    a = rounded(g.standard_normal((m, k)).astype(np.float32), kind)
    b = rounded(g.standard_normal((k, n)).astype(np.float32), kind)
    c = g.standard_normal((m, n)).astype(np.float32)
    a[3, 5] = np.nan
    b[7, 9] = np.inf
    c[10, 11] = -np.inf
    ref = oracle.gemm_f64(a, b, c, 1.0, 0.0)  # beta = 0 with c: 0 * -inf = NaN propagates
    at, bt = torch.from_numpy(a).to(DT[kind]).cuda(), torch.from_numpy(b).to(DT[kind]).cuda()
    ct = torch.from_numpy(c).cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(at, bt, ct, d, 1.0, 0.0, ops)
    for i in range(len(plan)):
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        rep = oracle.tolerance_check(d.cpu().numpy(), ref, k)
        assert rep["ok"], (plan.name(i), rep)


def test_half_type_rules(capi, ops):
    x = torch.zeros(64, device="cuda")
    p = x.data_ptr()
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    V = capi.View
    # Mixed a / b types, and a half d with an fp32 c: nothing applies.
    for a_t, b_t, c_t, d_t, why in ((capi.BF16, capi.FP16, capi.FP32, capi.FP32, "a or b is not bf16"),
                                    (capi.BF16, capi.BF16, capi.FP32, capi.BF16, "c and d must both be")):
        args = ops.args(V(p, [3, 2], numeric_type=a_t), V(p, [2, 4], numeric_type=b_t),
                        V(p, [3, 4], numeric_type=c_t), V(p, [3, 4], numeric_type=d_t), al.view, be.view)
        with pytest.raises(capi.FTrainError) as e:
            args.plan()
        assert e.value.status == capi.UNSUPPORTED and why in e.value.message
    # fp16 a with fp32 b, c, d: the reference's own case, every fp32 Primitive says so.
    args = ops.args(V(p, [3, 2], numeric_type=capi.FP16), V(p, [2, 4]), V(p, [3, 4]), V(p, [3, 4]), al.view, be.view)
    with pytest.raises(capi.FTrainError) as e:
        args.plan()
    assert "Fp32Gemm" in e.value.message and "an operand is not fp32" in e.value.message


@pytest.mark.parametrize("kind", ["bf16", "fp16"])
def test_half_large_sampled(capi, ops, oracle, kind):
    # 4096^3 in the x @ W^T orientation (b column-major) on Primitive 0, sampled rows.
    m = n = k = 4096
    gen = torch.Generator().manual_seed(2026)
    a = torch.randn(m, k, generator=gen).to(DT[kind])
    w = torch.randn(n, k, generator=gen).to(DT[kind])  # b = w^T
    ad, wd = a.cuda(), w.cuda()
    d = torch.empty(m, n, device="cuda")
    plan = capi.plan_for(ad, wd.t(), None, d, 1.0, 0.0, ops)
    assert plan.name(0).startswith(kind.capitalize() + "MfmaGemm_256x256") or plan.name(0).startswith(
        kind.capitalize() + "MfmaGemm_128x128"), plan.names()
    plan.execute(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    rows = np.random.default_rng(1).choice(m, 64, replace=False)
    ref = oracle.gemm_f64(a.float().numpy()[rows], w.float().numpy().T, None, 1.0, 0.0)
    rep = oracle.tolerance_check(d.cpu().numpy()[rows], ref, k)
    assert rep["ok"], rep


@pytest.mark.parametrize("name", ["square_8192", "mlp_fwd", "skinny_64x4096x4096"])
def test_half_bench_configs_at_full_size(capi, ops, oracle, name):
    """The bf16 configurations the bench reports, at their full size (fp32 d): 64 sampled rows of the
    Finder's pick against fp64 of the decoded bf16 inputs, far inside the bar, and over every row the
    size-independent identity d @ 1 = alpha * a @ (b @ 1) + beta * c @ 1."""
    import math

    a_h, b_h, c_h, cfg = oracle.seeded_inputs(name)
    a_h, b_h = a_h.to(torch.bfloat16), b_h.to(torch.bfloat16)
    m, n, k, alpha, beta = cfg["m"], cfg["n"], cfg["k"], cfg["alpha"], cfg["beta"]
    d = torch.full((m, n), float("nan"), device="cuda")
    plan = capi.plan_for(a_h.cuda(), b_h.cuda(), c_h.cuda() if c_h is not None else None, d, alpha, beta, ops)
    print(name, plan.names()[:3])
    plan.execute(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(7).choice(m, size=min(m, 64), replace=False))
    ref = oracle.sampled_rows_f64(a_h.float(), b_h.float(), c_h, alpha, beta, rows)
    rep = oracle.tolerance_check(d[torch.as_tensor(rows).cuda()].cpu().numpy(), ref, k)
    assert rep["ok"] and rep["max_abs_err"] <= 1e-2 * rep["bound"], (name, plan.name(0), rep)
    row_sums = d.double().sum(dim=1).cpu()
    want = alpha * (a_h.double() @ b_h.double().sum(dim=1))
    if c_h is not None:
        want += beta * c_h.double().sum(dim=1)
    err = (row_sums - want).abs().max().item()
    scale = want.abs().max().item() + math.sqrt(n * k)
    assert err <= 1e-4 * math.sqrt(k) * scale, (name, err, scale)
