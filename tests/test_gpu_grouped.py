"""GPU parity of the grouped Gemm families, called through the C ABI.

Every group g computes d_g = alpha * (a_g @ b_g) + beta * c_g; each group is
compared with the fp64 oracle (oracle.gemm_f64) to the north-star bar
max|d - ref| <= 1e-4 * sqrt(k) * max|ref| (widened by a 16-bit d's rounding).
Operand addressing follows the reference's GroupedTensor rule
(include/flash_train/common.h:397-425): element (i, j) of group g sits at
offsets[g] + i * strides[0][g] + j * strides[1][g] from data.memory.  The
shapes mimic mixture-of-experts training: packed token rows per expert
(forward), one weight matrix per expert, and the weight gradient whose
reduction depth is each expert's token count (including zero).
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


def rnd(shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def run_all(capi, args, check):
    plan = args.plan()
    args.close()
    names = plan.names()
    for i, name in enumerate(names):
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        check(name)
    # The device parameter table is uploaded once; a second execution reuses it.
    plan.execute(0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    check(names[0])
    return names


def close(oracle, d, ref, k, out_type="fp32", what=""):
    rep = oracle.tolerance_check(d, ref, k, out_type)
    assert rep["ok"], (what, rep)


@pytest.mark.parametrize("dtype,dname", [(torch.float32, "fp32"), (torch.bfloat16, "bf16"), (torch.float16, "fp16")])
def test_abcd_moe_forward(capi, oracle, dtype, dname):
    m_list, k, n = [0, 128, 37, 256, 64, 129], 192, 160
    G, M = len(m_list), sum(m_list)
    a = rnd((M, k), 1, dtype).cuda()
    b = rnd((G, k, n), 2, dtype).cuda()
    c = rnd((M, n), 3).cuda()
    d = torch.full((M, n), float("nan"), device="cuda")
    alpha, beta = 1.25, -0.5
    ops = capi.GroupedOps("abcd")
    al, be = capi.HostScalar(alpha), capi.HostScalar(beta)
    spec = lambda t, dims: capi.GroupedSpec(capi.matrix(t.view(t.shape[0] if t.dim() == 2 else -1, t.shape[-1])), G,
                                            dims=dims)
    args = ops.args(a=spec(a, [(m, k) for m in m_list]), b=capi.GroupedSpec(capi.matrix(b[0]), G),
                    c=spec(c, [(m, n) for m in m_list]), d=spec(d, [(m, n) for m in m_list]),
                    alpha=al.view, beta=be.view)
    a_h, b_h, c_h = a.float().cpu().numpy(), b.float().cpu().numpy(), c.cpu().numpy()

    def check(name):
        d_h, row = d.cpu().numpy(), 0
        for g, m in enumerate(m_list):
            ref = oracle.gemm_f64(a_h[row:row + m], b_h[g], c_h[row:row + m], alpha, beta)
            close(oracle, d_h[row:row + m], ref, k, what=(name, g))
            row += m
        d.fill_(float("nan"))

    names = run_all(capi, args, check)
    assert names[0].startswith("Grouped" + dname.capitalize()), names


def test_abcd_half_output(capi, oracle):
    m_list, k, n = [64, 0, 96], 128, 64
    G, M = len(m_list), sum(m_list)
    a = rnd((M, k), 4, torch.bfloat16).cuda()
    b = rnd((G * k, n), 5, torch.bfloat16).cuda()
    c = rnd((M, n), 6, torch.bfloat16).cuda()
    d = torch.zeros(M, n, dtype=torch.bfloat16, device="cuda")
    ops = capi.GroupedOps("abcd")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.5)
    dims_mn = [(m, n) for m in m_list]
    args = ops.args(a=capi.GroupedSpec(capi.matrix(a), G, dims=[(m, k) for m in m_list]),
                    b=capi.GroupedSpec(capi.matrix(b, [k, n]), G),
                    c=capi.GroupedSpec(capi.matrix(c), G, dims=dims_mn),
                    d=capi.GroupedSpec(capi.matrix(d), G, dims=dims_mn), alpha=al.view, beta=be.view)
    a_h, b_h, c_h = a.float().cpu().numpy(), b.float().cpu().numpy(), c.float().cpu().numpy()

    def check(name):
        d_h, row = d.float().cpu().numpy(), 0
        for g, m in enumerate(m_list):
            ref = oracle.gemm_f64(a_h[row:row + m], b_h[g * k:(g + 1) * k], c_h[row:row + m], 1.0, 0.5)
            close(oracle, d_h[row:row + m], ref, k, "bf16", (name, g))
            row += m

    run_all(capi, args, check)


def test_bcd_tensor_list_with_mixed_orientations(capi, oracle):
    # a_0 row-major, a_1 a transposed view (column-major), a_2 row-major with odd rows.
    k, n = 96, 128
    a0 = rnd((64, k), 7).cuda()
    a1 = rnd((k, 48), 8).cuda().t()
    a2 = rnd((33, k), 9).cuda()
    a_list = [a0, a1, a2]
    m_list = [t.shape[0] for t in a_list]
    G, M = 3, sum(m_list)
    b = rnd((G * k, n), 10).cuda()
    d = torch.full((M, n), float("nan"), device="cuda")
    ops = capi.GroupedOps("bcd")
    al, be = capi.HostScalar(2.0), capi.HostScalar(0.0)
    dims = [(m, n) for m in m_list]
    args = ops.args(a=[capi.matrix(t) for t in a_list], b=capi.GroupedSpec(capi.matrix(b, [k, n]), G),
                    c=capi.GroupedSpec(capi.View(None, [M, n]), G, dims=dims),
                    d=capi.GroupedSpec(capi.matrix(d), G, dims=dims), alpha=al.view, beta=be.view)
    b_h = b.cpu().numpy()

    def check(name):
        d_h, row = d.cpu().numpy(), 0
        for g, t in enumerate(a_list):
            m = t.shape[0]
            ref = oracle.gemm_f64(t.cpu().numpy(), b_h[g * k:(g + 1) * k], None, 2.0, 0.0)
            close(oracle, d_h[row:row + m], ref, k, what=(name, g))
            row += m
        d.fill_(float("nan"))

    run_all(capi, args, check)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ab_weight_gradient(capi, oracle, dtype):
    # dW_g = X_g^T @ dY_g over each expert's tokens: k_g = tokens (0 included: dW_g = beta * c_g).
    tokens, M, N = [40, 0, 24, 130], 64, 96
    G, T = len(tokens), sum(tokens)
    X = rnd((T, M), 11, dtype).cuda()
    dY = rnd((T, N), 12, dtype).cuda()
    c_list = [rnd((M, N), 20 + g).cuda() for g in range(G)]
    d_list = [torch.full((M, N), float("nan"), device="cuda") for _ in range(G)]
    offs = [sum(tokens[:g]) for g in range(G)]
    ops = capi.GroupedOps("ab")
    al, be = capi.HostScalar(1.0), capi.HostScalar(1.0)
    args = ops.args(
        a=capi.GroupedSpec(capi.matrix(X), G, dims=[(M, t) for t in tokens], strides=[(1, M)] * G,
                           offsets=[o * M for o in offs]),
        b=capi.GroupedSpec(capi.matrix(dY), G, dims=[(t, N) for t in tokens]),
        c=[capi.matrix(t) for t in c_list], d=[capi.matrix(t) for t in d_list], alpha=al.view, beta=be.view)
    X_h, dY_h = X.float().cpu().numpy(), dY.float().cpu().numpy()

    def check(name):
        for g, t in enumerate(tokens):
            o = offs[g]
            ref = oracle.gemm_f64(np.ascontiguousarray(X_h[o:o + t].T), dY_h[o:o + t], c_list[g].cpu().numpy(), 1.0,
                                  1.0)
            close(oracle, d_list[g].cpu().numpy(), ref, max(t, 1), what=(name, g))
            d_list[g].fill_(float("nan"))

    run_all(capi, args, check)


def test_abcd_explicit_offsets_and_padded_strides(capi, oracle):
    # Groups placed out of order with gaps inside NaN-filled storage, each with a padded leading dimension.
    k, n = 64, 96
    m_list = [48, 80]
    pad = 8
    store_a = torch.full((4096 * 4,), float("nan"), device="cuda")
    store_d = torch.full((4096 * 8,), 7.0, device="cuda")
    a_groups = [rnd((m, k), 30 + g) for g, m in enumerate(m_list)]
    a_offs, d_offs = [9000, 256], [20000, 64]
    for g, m in enumerate(m_list):
        view = store_a[a_offs[g]:a_offs[g] + m * (k + pad)].view(m, k + pad)
        view[:, :k] = a_groups[g].cuda()
    b = rnd((k, n), 40).cuda()
    ops = capi.GroupedOps("abcd")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    G = 2
    args = ops.args(
        a=capi.GroupedSpec(capi.matrix(store_a.view(-1, 1)), G, dims=[(m, k) for m in m_list],
                           strides=[(k + pad, 1)] * G, offsets=a_offs),
        b=capi.GroupedSpec(capi.View(b.data_ptr(), [k, n]), G, offsets=[0, 0]),
        c=capi.GroupedSpec(capi.View(None, [1, 1]), G, dims=[(m, n) for m in m_list]),
        d=capi.GroupedSpec(capi.matrix(store_d.view(-1, 1)), G, dims=[(m, n) for m in m_list],
                           strides=[(n + pad, 1)] * G, offsets=d_offs),
        alpha=al.view, beta=be.view)
    b_h = b.cpu().numpy()

    def check(name):
        sd = store_d.cpu().numpy()
        touched = np.zeros(sd.shape, bool)
        for g, m in enumerate(m_list):
            ref = oracle.gemm_f64(a_groups[g].numpy(), b_h, None, 1.0, 0.0)
            idx = d_offs[g] + np.arange(m)[:, None] * (n + pad) + np.arange(n)[None, :]
            close(oracle, sd[idx], ref, k, what=(name, g))
            touched[idx] = True
        assert np.all(sd[~touched] == 7.0), (name, "wrote outside the groups")
        store_d.fill_(7.0)

    run_all(capi, args, check)


def test_many_small_groups(capi, oracle):
    # 300 groups of 0-40 rows: the workgroup -> group binary search over
    # hundreds of tile starts, every tile padded to its group's XCD slot.
    rng = np.random.default_rng(7)
    G, k, n = 300, 32, 48
    m_list = [int(x) for x in rng.integers(0, 41, size=G)]
    M = sum(m_list)
    a = rnd((M, k), 50).cuda()
    b = rnd((G * k, n), 51).cuda()
    d = torch.full((M, n), float("nan"), device="cuda")
    ops = capi.GroupedOps("abcd")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    dims = [(m, n) for m in m_list]
    args = ops.args(a=capi.GroupedSpec(capi.matrix(a), G, dims=[(m, k) for m in m_list]),
                    b=capi.GroupedSpec(capi.matrix(b, [k, n]), G),
                    c=capi.GroupedSpec(capi.View(None, [M, n]), G, dims=dims),
                    d=capi.GroupedSpec(capi.matrix(d), G, dims=dims), alpha=al.view, beta=be.view)
    a_h, b_h = a.cpu().numpy(), b.cpu().numpy()

    def check(name):
        d_h, row = d.cpu().numpy(), 0
        for g, m in enumerate(m_list):
            ref = oracle.gemm_f64(a_h[row:row + m], b_h[g * k:(g + 1) * k], None, 1.0, 0.0)
            close(oracle, d_h[row:row + m], ref, k, what=(name, g))
            row += m
        d.fill_(float("nan"))

    run_all(capi, args, check)


def test_no_groups_and_all_empty_groups_launch_nothing(capi):
    k, n = 32, 48
    sentinel = torch.full((8, n), 3.0, device="cuda")
    for m_list in ([], [0, 0, 0]):
        G = len(m_list)
        ops = capi.GroupedOps("abcd")
        al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
        dims = [(m, n) for m in m_list]
        args = ops.args(a=capi.GroupedSpec(capi.matrix(sentinel[:, :k].contiguous()), G, dims=[(m, k) for m in m_list]),
                        b=capi.GroupedSpec(capi.View(sentinel.data_ptr(), [k, n]), G),
                        c=capi.GroupedSpec(capi.View(None, [8, n]), G, dims=dims),
                        d=capi.GroupedSpec(capi.matrix(sentinel), G, dims=dims), alpha=al.view, beta=be.view)
        plan = args.plan()
        args.close()
        for i in range(len(plan)):
            plan.execute(i)
        torch.cuda.synchronize()
        assert torch.all(sentinel == 3.0), m_list


def test_abcd_column_major_weights(capi, oracle):
    """Per-expert weights stored as nn.Linear keeps them (n x k, so b_g is a column-major view):
    every fp32 grouped Primitive, edge rows and columns, against fp64."""
    m_list, k, n = [300, 0, 129, 512], 256, 200
    G, M = len(m_list), sum(m_list)
    a = rnd((M, k), 21).cuda()
    w = rnd((G, n, k), 22).cuda()  # storage of b_g^T
    c = rnd((M, n), 23).cuda()
    d = torch.full((M, n), float("nan"), device="cuda")
    ops = capi.GroupedOps("abcd")
    al, be = capi.HostScalar(0.5), capi.HostScalar(2.0)
    dims = [(m, n) for m in m_list]
    args = ops.args(a=capi.GroupedSpec(capi.matrix(a), G, dims=[(m, k) for m in m_list]),
                    b=capi.GroupedSpec(capi.matrix(w.view(G * n, k)), G, dims=[(k, n)] * G, strides=[(1, k)] * G,
                                       offsets=[g * n * k for g in range(G)]),
                    c=capi.GroupedSpec(capi.matrix(c), G, dims=dims), d=capi.GroupedSpec(capi.matrix(d), G, dims=dims),
                    alpha=al.view, beta=be.view)
    a_h, w_h, c_h = a.cpu().numpy(), w.cpu().numpy(), c.cpu().numpy()

    def check(name):
        d_h, row = d.cpu().numpy(), 0
        for g, m in enumerate(m_list):
            ref = oracle.gemm_f64(a_h[row:row + m], w_h[g].T.copy(), c_h[row:row + m], 0.5, 2.0)
            close(oracle, d_h[row:row + m], ref, k, what=(name, g))
            row += m
        d.fill_(float("nan"))

    names = run_all(capi, args, check)
    assert "GroupedFp32Mfma16Gemm_128x128_Dma" in names, names


@pytest.mark.parametrize("dtype,dname", [(torch.bfloat16, "Bf16"), (torch.float16, "Fp16")])
@pytest.mark.parametrize("b_col_major", [False, True])
def test_abcd_half_large_total_b_exact(capi, dtype, dname, b_col_major):
    """Eight experts whose weights total 302 MB (each 4096 x 4616, 16-bit, row-major or stored as
    nn.Linear keeps them) and at least 8 tile rows each: the grouped 256x256 DMA tile then prefetches
    b into L2.  n = 18 * 256 + 8 leaves a last column tile of 8 (prefetched lines clamped onto the
    matrix).  Integer inputs in [-2, 2] make every fp32 result exact, so each group must equal its
    fp64 product bit for bit, ragged rows and an empty group included."""
    m_list, k, n = [2085, 0, 2100, 1999, 2300, 2048, 2200, 1900, 2171], 4096, 4616
    G, M = len(m_list), sum(m_list)
    gen = torch.Generator(device="cuda").manual_seed(31)
    a = torch.randint(-2, 3, (M, k), device="cuda", generator=gen).to(dtype)
    b = torch.randint(-2, 3, (G, k, n), device="cuda", generator=gen).to(dtype)
    d = torch.full((M, n), float("nan"), device="cuda")
    ops = capi.GroupedOps("abcd")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    dims = [(m, n) for m in m_list]
    if b_col_major:
        w = b.transpose(1, 2).contiguous()  # storage of b_g^T, n x k per group
        bspec = capi.GroupedSpec(capi.matrix(w.view(G * n, k)), G, dims=[(k, n)] * G, strides=[(1, k)] * G,
                                 offsets=[g * n * k for g in range(G)])
    else:
        bspec = capi.GroupedSpec(capi.matrix(b.view(G * k, n)), G, dims=[(k, n)] * G)
    args = ops.args(a=capi.GroupedSpec(capi.matrix(a), G, dims=[(m, k) for m in m_list]), b=bspec,
                    c=capi.GroupedSpec(capi.View(None, [M, n], numeric_type=capi.TORCH_NUMERIC_TYPES[torch.float32]), G,
                                       dims=dims),
                    d=capi.GroupedSpec(capi.matrix(d), G, dims=dims), alpha=al.view, beta=be.view)
    plan = args.plan()
    args.close()
    names = plan.names()
    i = names.index(f"Grouped{dname}MfmaGemm_256x256_Dma")
    want, row = [], 0
    for g, m in enumerate(m_list):
        want.append((a[row:row + m].double() @ b[g].double()).float())
        row += m
    if b_col_major:
        del b
    for _ in range(2):
        d.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        row = 0
        for g, m in enumerate(m_list):
            assert torch.equal(d[row:row + m], want[g]), (g, m)
            row += m


@pytest.mark.parametrize("dtype,dname", [(torch.bfloat16, "Bf16"), (torch.float16, "Fp16")])
def test_ab_weight_gradient_ragged_tokens_exact_on_dma_tiles(capi, dtype, dname):
    """dW_g = X_g^T @ dY_g with token counts that are not multiples of 64 (one below a stage, one of
    zero): every Primitive of the Plan, the DMA tiles included (their partial last stage staged by
    ordinary loads, zeros past each expert's tokens).  Integer inputs in [-2, 2] make the fp32
    result exact, so each group must equal its fp64 product bit for bit."""
    tokens, M, N = [1000, 0, 37, 300, 129, 2100], 512, 768
    G, T = len(tokens), sum(tokens)
    gen = torch.Generator(device="cuda").manual_seed(41)
    X = torch.randint(-2, 3, (T, M), device="cuda", generator=gen).to(dtype)
    dY = torch.randint(-2, 3, (T, N), device="cuda", generator=gen).to(dtype)
    d_list = [torch.full((M, N), float("nan"), device="cuda") for _ in range(G)]
    offs = [sum(tokens[:g]) for g in range(G)]
    ops = capi.GroupedOps("ab")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    args = ops.args(
        a=capi.GroupedSpec(capi.matrix(X), G, dims=[(M, t) for t in tokens], strides=[(1, M)] * G,
                           offsets=[o * M for o in offs]),
        b=capi.GroupedSpec(capi.matrix(dY), G, dims=[(t, N) for t in tokens]),
        c=[capi.View(None, [M, N], numeric_type=capi.TORCH_NUMERIC_TYPES[torch.float32]) for _ in range(G)],
        d=[capi.matrix(t) for t in d_list], alpha=al.view, beta=be.view)
    plan = args.plan()
    args.close()
    names = plan.names()
    assert f"Grouped{dname}MfmaGemm_256x256_Dma" in names and f"Grouped{dname}MfmaGemm_128x128_Dma" in names, names
    want = [(X[o:o + t].double().t() @ dY[o:o + t].double()).float() for o, t in zip(offs, tokens)]
    for i, name in enumerate(names):
        for t in d_list:
            t.fill_(float("nan"))
        plan.execute(i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        for g in range(G):
            assert torch.equal(d_list[g], want[g]), (name, g, tokens[g])


def test_ab_weight_gradient_ragged_tokens_fp32_dma_tile(capi, oracle):
    """fp32 dW_g = X_g^T @ dY_g with token counts that are not multiples of 32 (one of zero, one below a
    stage): every Primitive, the 128x128 DMA tile included (partial last stage staged by ordinary
    loads), against fp64."""
    tokens, M, N = [500, 0, 19, 300, 129], 256, 384
    G, T = len(tokens), sum(tokens)
    X = rnd((T, M), 51).cuda()
    dY = rnd((T, N), 52).cuda()
    d_list = [torch.full((M, N), float("nan"), device="cuda") for _ in range(G)]
    offs = [sum(tokens[:g]) for g in range(G)]
    ops = capi.GroupedOps("ab")
    al, be = capi.HostScalar(1.0), capi.HostScalar(0.0)
    args = ops.args(
        a=capi.GroupedSpec(capi.matrix(X), G, dims=[(M, t) for t in tokens], strides=[(1, M)] * G,
                           offsets=[o * M for o in offs]),
        b=capi.GroupedSpec(capi.matrix(dY), G, dims=[(t, N) for t in tokens]),
        c=[capi.View(None, [M, N]) for _ in range(G)], d=[capi.matrix(t) for t in d_list], alpha=al.view,
        beta=be.view)
    X_h, dY_h = X.cpu().numpy(), dY.cpu().numpy()

    def check(name):
        for g, t in enumerate(tokens):
            o = offs[g]
            ref = oracle.gemm_f64(np.ascontiguousarray(X_h[o:o + t].T), dY_h[o:o + t], None, 1.0, 0.0)
            close(oracle, d_list[g].cpu().numpy(), ref, max(t, 1), what=(name, g))
            d_list[g].fill_(float("nan"))

    names = run_all(capi, args, check)
    assert "GroupedFp32Mfma16Gemm_128x128_Dma" in names, names
