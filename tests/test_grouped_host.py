"""Host-side contract of the grouped Gemm families -- no GPU needed.

The reference declares GroupedABCDGemm, GroupedBCDGemm and GroupedABGemm with
their operand storage families (src/include/flash_train/operation/gemm.hpp:80-150)
and the GroupedTensor addressing rule (include/flash_train/common.h:397-425),
but registers no engine for them.  These tests pin this build's engines:
Pattern matching, per-group validation statuses, descriptor support checks,
and which Primitives apply.  Plan creation goes through the testing hook with
fake device addresses (never dereferenced before execution).
"""

import ctypes

import pytest

from flash_train import capi as c

FAKE = 0x7F0000000000


@pytest.fixture(scope="module")
def tlib():
    return c.testing_lib()


def D(dims, mem=FAKE, **kw):
    return c.View(mem, dims, **kw)


def scalars():
    al, be = c.HostScalar(1.5), c.HostScalar(0.5)
    return al, be


def moe_abcd(tlib, m_list, k=64, n=96, a_type=c.FP32, d_type=None, b_dims=None, dev_desc=False, a_strides=None,
             mem=FAKE):
    """ABCD args: a packed [sum m, k], b one [k, n] per group, c and d packed [sum m, n]."""
    d_type = d_type or (a_type if a_type == c.FP32 else c.FP32)
    G = len(m_list)
    ops = c.GroupedOps("abcd", l=tlib)
    spec = lambda rows_cols, t, strides=None: c.GroupedSpec(D([max(sum(r for r, _ in rows_cols), 1), 1], mem,
                                                              numeric_type=t), G, dims=rows_cols, strides=strides)
    a = spec([(m, k) for m in m_list], a_type, a_strides)
    b = spec(b_dims or [(k, n)] * G, a_type)
    cc = spec([(m, n) for m in m_list], d_type)
    d = spec([(m, n) for m in m_list], d_type)
    if dev_desc:
        a.dim_views[0].is_host_memory = False
    al, be = scalars()
    args = ops.args(a=a, b=b, c=cc, d=d, alpha=al.view, beta=be.view)
    st, msg, plan = args.plan_status_on_device(0)
    return st, msg, plan


def test_every_grouped_kind_gets_an_ops(tlib):
    for kind in ("abcd", "bcd", "ab"):
        ops = c.GroupedOps(kind, l=tlib)
        assert ops.ops
        ops.close()


FP32_GROUPED = ["GroupedFp32Mfma16Gemm_256x256_Dma", "GroupedFp32Mfma16Gemm_128x128_Dma", "GroupedFp32Mfma16Gemm_64x128_Dma",
                "GroupedFp32Mfma16Gemm_256x128",
                "GroupedFp32Mfma16Gemm_128x256", "GroupedFp32MfmaGemm_128x128", "GroupedFp32MfmaGemm_64x64_Unaligned"]


def test_abcd_plan_and_primitive_order(tlib):
    # Few, small groups: every fp32 tile applies; the cost model puts the
    # smallest tile first (most workgroups for 256 CUs).
    st, msg, plan = moe_abcd(tlib, [128, 0, 37, 256])
    assert st == c.SUCCESS, msg
    assert sorted(plan.names()) == sorted(FP32_GROUPED)
    assert plan.names()[0] == "GroupedFp32MfmaGemm_64x64_Unaligned"
    assert all(plan.workspace_bytes(i) == 0 for i in range(len(plan)))


def test_large_groups_take_the_large_tiles(tlib):
    # Mixture-of-experts forward: 8 experts over 16384 tokens, k 4096, n 14336.
    rows = [2100, 1900, 2300, 1700, 2048, 2200, 1800, 2336]
    st, msg, plan = moe_abcd(tlib, rows, k=4096, n=14336)
    assert st == c.SUCCESS, msg
    assert plan.names()[0] in ("GroupedFp32Mfma16Gemm_256x256_Dma", "GroupedFp32Mfma16Gemm_128x128_Dma",
                               "GroupedFp32Mfma16Gemm_128x256")
    st, msg, plan = moe_abcd(tlib, rows, k=4096, n=14336, a_type=c.BF16)
    assert st == c.SUCCESS, msg
    assert plan.names()[0] == "GroupedBf16MfmaGemm_256x256_Dma"


def test_disabled_grouped_finder_falls_back_to_registration_order():
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    prog = ("import sys; sys.path[:0]=[%r, %r, %r]\n" % (os.path.join(repo, "flash-train_amd"), repo,
                                                        os.path.join(repo, "tests")) +
            "from test_grouped_host import moe_abcd\nfrom flash_train import capi as c\n"
            "st, msg, plan = moe_abcd(c.testing_lib(), [128, 0, 37, 256])\nprint(','.join(plan.names()))")
    out = subprocess.run([sys.executable, "-c", prog], env=dict(os.environ, FTRAIN_DISABLED_FINDERS="GroupedCost"),
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip().split(",") == FP32_GROUPED


def test_unaligned_groups_take_the_per_element_tile(tlib):
    st, msg, plan = moe_abcd(tlib, [16, 8], k=33, n=96)
    assert st == c.SUCCESS, msg
    assert plan.names() == ["GroupedFp32MfmaGemm_64x64_Unaligned"]


def test_half_types_select_their_variants(tlib):
    st, msg, plan = moe_abcd(tlib, [64, 32], a_type=c.BF16)
    assert st == c.SUCCESS, msg
    assert sorted(plan.names()) == sorted(["GroupedBf16MfmaGemm_256x256_Dma", "GroupedBf16MfmaGemm_128x128_Dma",
                                           "GroupedBf16MfmaGemm_256x256", "GroupedBf16MfmaGemm_128x128",
                                           "GroupedBf16MfmaGemm_64x64_Unaligned"])
    st, msg, plan = moe_abcd(tlib, [64, 32], a_type=c.FP16, d_type=c.FP16)
    assert st == c.SUCCESS, msg
    assert all(n.startswith("GroupedFp16") for n in plan.names()) and len(plan) == 5
    # k not a multiple of 64: the DMA tiles stage the partial last stage themselves and stay.
    st, msg, plan = moe_abcd(tlib, [64, 32], k=72, a_type=c.BF16)
    assert st == c.SUCCESS, msg
    assert "GroupedBf16MfmaGemm_256x256_Dma" in plan.names() and len(plan) == 5
    # k not a multiple of 8 with a k-contiguous operand: 16-byte loads do not fit, only the
    # per-element tile remains.
    st, msg, plan = moe_abcd(tlib, [64, 32], k=70, a_type=c.BF16)
    assert st == c.SUCCESS, msg
    assert plan.names() == ["GroupedBf16MfmaGemm_64x64_Unaligned"]


def test_group_shape_mismatch_is_invalid(tlib):
    st, msg, _ = moe_abcd(tlib, [64, 32], b_dims=[(64, 96), (63, 96)])
    assert st == c.INVALID_ARGUMENT and "group 1" in msg, msg


def test_device_descriptors_are_unsupported(tlib):
    st, msg, _ = moe_abcd(tlib, [64, 32], dev_desc=True)
    assert st == c.UNSUPPORTED and "host memory" in msg, msg


def test_mixed_orientations_are_accepted(tlib):
    # Group 0 row-major, group 1 column-major a: one launch per orientation.
    st, msg, plan = moe_abcd(tlib, [64, 32], a_strides=[(64, 1), (1, 32)])
    assert st == c.SUCCESS, msg
    # the 256x256 fp32 DMA tile takes row-major a and b only, the 64x128 one row-major a
    assert sorted(plan.names()) == sorted(n for n in FP32_GROUPED if n not in FP32_GROUPED[0:3:2])


def test_group_count_mismatch_is_invalid(tlib):
    ops = c.GroupedOps("abcd", l=tlib)
    a = c.GroupedSpec(D([256, 64]), 2, dims=[(128, 64), (128, 64)])
    b = c.GroupedSpec(D([64, 96]), 3)
    cd = c.GroupedSpec(D([256, 96]), 2, dims=[(128, 96), (128, 96)])
    al, be = scalars()
    st, msg, _ = ops.args(a=a, b=b, c=cd, d=cd, alpha=al.view, beta=be.view).plan_status_on_device(0)
    assert st == c.INVALID_ARGUMENT and "groups" in msg, msg


def test_descriptor_types_and_values(tlib):
    ops = c.GroupedOps("abcd", l=tlib)
    al, be = scalars()
    bad = c.GroupedSpec(D([256, 64]), 2, dims=[(128, 64), (128, 64)])
    bad.dim_views[0].numeric_type = c.FP32
    b = c.GroupedSpec(D([64, 96]), 2)
    cd = c.GroupedSpec(D([256, 96]), 2, dims=[(128, 96), (128, 96)])
    st, msg, _ = ops.args(a=bad, b=b, c=cd, d=cd, alpha=al.view, beta=be.view).plan_status_on_device(0)
    assert st == c.UNSUPPORTED and "int32" in msg, msg
    neg = c.GroupedSpec(D([256, 64]), 2, dims=[(128, 64), (-1, 64)])
    st, msg, _ = ops.args(a=neg, b=b, c=cd, d=cd, alpha=al.view, beta=be.view).plan_status_on_device(0)
    assert st == c.INVALID_ARGUMENT and "negative" in msg, msg


def test_bcd_with_a_tensor_list(tlib):
    ops = c.GroupedOps("bcd", l=tlib)
    al, be = scalars()
    a = [D([64, 48]), D([16, 48])]
    b = c.GroupedSpec(D([48, 32]), 2)
    cd = c.GroupedSpec(D([80, 32]), 2, dims=[(64, 32), (16, 32)])
    st, msg, plan = ops.args(a=a, b=b, c=cd, d=cd, alpha=al.view, beta=be.view).plan_status_on_device(0)
    assert st == c.SUCCESS, msg
    st, msg, _ = ops.args(a=a[:1], b=b, c=cd, d=cd, alpha=al.view, beta=be.view).plan_status_on_device(0)
    assert st == c.INVALID_ARGUMENT, msg


def test_ab_with_c_and_d_lists_and_a_column_major(tlib):
    # Weight-gradient form: a_g = X_g^T (column-major view of the packed tokens), k_g = tokens of group g.
    ops = c.GroupedOps("ab", l=tlib)
    al, be = scalars()
    tokens = [40, 0, 24]
    M, N = 64, 32
    a = c.GroupedSpec(D([sum(tokens), M]), 3, dims=[(M, t) for t in tokens], strides=[(1, M)] * 3,
                      offsets=[sum(tokens[:g]) * M for g in range(3)])
    b = c.GroupedSpec(D([sum(tokens), N]), 3, dims=[(t, N) for t in tokens])
    cl = [D([M, N]) for _ in tokens]
    st, msg, plan = ops.args(a=a, b=b, c=cl, d=cl, alpha=al.view, beta=be.view).plan_status_on_device(0)
    assert st == c.SUCCESS, msg
    # k of 40, 0 and 24 (partial stages): the 128x128 DMA tile takes any orientation; the 256x256
    # and 64x128 ones need a row-major a.
    assert sorted(plan.names()) == sorted(["GroupedFp32Mfma16Gemm_128x128_Dma"] + FP32_GROUPED[3:])


def test_descriptor_values_that_overflow_addresses_are_rejected(tlib):
    # Offsets or packed extents past the addressable range report OVERFLOW
    # instead of forming wrapped pointers.
    G, k, n = 2, 64, 96
    al, be = scalars()

    def status(a_spec):
        ops = c.GroupedOps("abcd", l=tlib)
        b = c.GroupedSpec(D([G * k, n]), G, dims=[(k, n)] * G)
        cd = lambda: c.GroupedSpec(D([128, n]), G, dims=[(64, n)] * G)
        args = ops.args(a=a_spec, b=b, c=cd(), d=cd(), alpha=al.view, beta=be.view)
        st, msg, _ = args.plan_status_on_device(0)
        return st, msg

    huge = 1 << 61
    st, msg = status(c.GroupedSpec(D([128, k]), G, dims=[(64, k)] * G, offsets=[0, huge]))
    assert st == c.OVERFLOW and "offsets[1]" in msg, msg
    st, msg = status(c.GroupedSpec(D([128, k]), G, dims=[(64, k)] * G, offsets=[0, (1 << 60) - 64]))
    assert st == c.OVERFLOW and "extent" in msg, msg
    # Packed groups (no offsets) whose sizes overflow the running offset.
    st, msg = status(c.GroupedSpec(D([128, k]), G, dims=[(1 << 40, 1 << 40), (64, k)]))
    assert st == c.OVERFLOW and "packed" in msg, msg
