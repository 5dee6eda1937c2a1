"""Host-side contract of the C ABI -- no GPU needed.

Mirrors the reference's host tests: tests/api/common_api_test.cpp (thread
local status), tests/api/pattern_api_test.cpp and tests/pattern_test.cpp
(Pattern validation), tests/matcher_test.cpp (order-insensitive matching),
tests/storage_view_test.cpp, tests/tensor_test.cpp, tests/ops_args_test.cpp,
tests/api/gemm_api_test.cpp:140-328 (plan-creation statuses),
tests/cache/cache_test.cpp and tests/engine/engine_test.cpp (selection cache,
environment filters).  Plan creation on a CPU host goes through the test
hook ftrainTestingPlanCreateOnDevice (libflash_train_testing.so), which runs
the same engine for an explicit device id; addresses are never dereferenced
before execution, so fake device addresses are used.
"""

import ctypes
import os
import shutil
import subprocess
import sys
import threading

import pytest

from flash_train import capi as c

FAKE = 0x7F0000000000  # 16-byte aligned stand-in device address (never dereferenced)


@pytest.fixture(scope="module")
def lib():
    return c.lib()


@pytest.fixture(scope="module")
def tlib():
    return c.testing_lib()


# ------------------------------------------------------------------ library


def test_library_exports_exactly_the_reference_symbols():
    assert os.path.exists(c.LIBRARY_PATH)
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", c.LIBRARY_PATH], capture_output=True, text=True).stdout
    exported = sorted(line.split()[-1] for line in out.splitlines() if line.split() and line.split()[1] in "TW")
    assert exported == sorted(c.EXPORTED_SYMBOLS)


def test_every_declared_symbol_resolves(lib):
    for name in c.EXPORTED_SYMBOLS:
        assert getattr(lib, name) is not None


def test_header_declares_every_exported_symbol():
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = open(os.path.join(repo, "include", "flash_train", "common.h")).read()
    text += open(os.path.join(repo, "include", "flash_train", "flash_train.h")).read()
    for name in c.EXPORTED_SYMBOLS:
        assert f" {name}(" in text, name


# ------------------------------------------------------------------ thread-local status


def test_last_status_semantics(lib):
    p = ctypes.c_void_p()
    assert lib.ftrainPatternCreate(None) == c.INVALID_ARGUMENT
    assert lib.ftrainGetLastStatus() == c.INVALID_ARGUMENT
    msg = lib.ftrainGetLastMessage()
    assert b"must not be null" in msg
    # Queries do not change the recorded result.
    assert lib.ftrainGetLastStatus() == c.INVALID_ARGUMENT
    assert lib.ftrainGetLastMessage() == msg
    # Success clears it.
    assert lib.ftrainPatternCreate(ctypes.byref(p)) == c.SUCCESS
    assert lib.ftrainGetLastStatus() == c.SUCCESS and lib.ftrainGetLastMessage() == b""
    assert lib.ftrainPatternDestroy(p) == c.SUCCESS


def test_last_status_is_per_thread(lib):
    assert lib.ftrainPatternDestroy(None) == c.INVALID_ARGUMENT
    seen = {}

    def worker():
        seen["fresh"] = (lib.ftrainGetLastStatus(), lib.ftrainGetLastMessage())
        lib.ftrainOpsDestroy(None)
        seen["after"] = lib.ftrainGetLastStatus()

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert seen["fresh"] == (c.SUCCESS, b"")
    assert seen["after"] == c.INVALID_ARGUMENT
    assert lib.ftrainGetLastStatus() == c.INVALID_ARGUMENT
    assert b"ftrainPatternDestroy" in lib.ftrainGetLastMessage()


def test_null_handles_rejected(lib):
    h = ctypes.c_void_p()
    n = ctypes.c_uint64(77)
    s = ctypes.c_char_p()
    rid = c.RoleId(5)
    assert lib.ftrainOpsCreate(ctypes.byref(h), None) == c.INVALID_ARGUMENT
    assert lib.ftrainOpsCreate(None, None) == c.INVALID_ARGUMENT
    assert lib.ftrainArgsCreate(ctypes.byref(h), None) == c.INVALID_ARGUMENT
    assert lib.ftrainArgsDestroy(None) == c.INVALID_ARGUMENT
    assert lib.ftrainArgsSetTensor(None, rid, c.View(FAKE, [2, 2]).sv) == c.INVALID_ARGUMENT
    assert lib.ftrainArgsSetGemm(None, rid, c.FP32) == c.INVALID_ARGUMENT
    assert lib.ftrainPlanCreate(ctypes.byref(h), None) == c.INVALID_ARGUMENT
    assert lib.ftrainPlanDestroy(None) == c.INVALID_ARGUMENT
    assert lib.ftrainPlanGetNumPrimitives(None, ctypes.byref(n)) == c.INVALID_ARGUMENT and n.value == 77
    assert lib.ftrainPlanGetPrimitiveName(None, 0, ctypes.byref(s)) == c.INVALID_ARGUMENT and s.value is None
    assert lib.ftrainPlanGetPrimitiveRequiredWorkspaceBytes(None, 0, ctypes.byref(n)) == c.INVALID_ARGUMENT
    assert lib.ftrainPlanExecutePrimitive(None, 0, None, 0, None) == c.INVALID_ARGUMENT
    assert h.value is None


# ------------------------------------------------------------------ Pattern / Ops


def new_pattern(lib):
    p = ctypes.c_void_p()
    c.check(lib.ftrainPatternCreate(ctypes.byref(p)), l=lib)
    return p


def add_tensors(lib, p, n):
    ids = []
    for _ in range(n):
        r = c.RoleId()
        c.check(lib.ftrainPatternAddTensor(p, ctypes.byref(r)), l=lib)
        ids.append(r)
    return ids


def ops_status(lib, p):
    o = ctypes.c_void_p()
    st = lib.ftrainOpsCreate(ctypes.byref(o), p)
    if st == c.SUCCESS:
        lib.ftrainOpsDestroy(o)
    else:
        assert o.value is None
    return st


def test_role_ids_are_sequential_and_outputs_untouched_on_failure(lib):
    p = new_pattern(lib)
    t, tl, gt = c.RoleId(99), c.RoleId(99), c.RoleId(99)
    assert lib.ftrainPatternAddTensor(p, ctypes.byref(t)) == c.SUCCESS
    assert lib.ftrainPatternAddTensorList(p, ctypes.byref(tl)) == c.SUCCESS
    assert lib.ftrainPatternAddGroupedTensor(p, ctypes.byref(gt)) == c.SUCCESS
    assert (t.opaque, tl.opaque, gt.opaque) == (0, 1, 2)
    probe = c.RoleId(73)
    assert lib.ftrainPatternAddTensor(None, ctypes.byref(probe)) == c.INVALID_ARGUMENT
    assert probe.opaque == 73
    lib.ftrainPatternDestroy(p)


@pytest.mark.parametrize("order", [(0, 1, 2, 3, 4, 5), (5, 4, 3, 2, 1, 0), (3, 0, 5, 1, 4, 2)])
def test_gemm_pattern_matches_in_any_insertion_order(lib, order):
    p = new_pattern(lib)
    ids = add_tensors(lib, p, 6)
    a, b, cc, d, al, be = [ids[i] for i in order]
    op = c.RoleId()
    assert lib.ftrainPatternAddGemm(p, ctypes.byref(op), a, b, cc, d, al, be) == c.SUCCESS
    assert ops_status(lib, p) == c.SUCCESS
    lib.ftrainPatternDestroy(p)


@pytest.mark.parametrize("ports,status", [
    ((0, 0, 2, 3, 4, 5), c.INVALID_ARGUMENT),   # repeated input
    ((0, 1, 2, 0, 4, 5), c.INVALID_ARGUMENT),   # output reuses an input
    ((0, 1, 2, 6, 4, 5), c.INVALID_ARGUMENT),   # out-of-range operand (id 9)
])
def test_conflicting_structures_are_rejected_when_built(lib, ports, status):
    p = new_pattern(lib)
    ids = add_tensors(lib, p, 6)
    ids.append(c.RoleId(9))
    op = c.RoleId(83)
    # Appending never validates (reference pattern_api_test.cpp:171-186).
    assert lib.ftrainPatternAddGemm(p, ctypes.byref(op), *[ids[i] for i in ports]) == c.SUCCESS
    assert ops_status(lib, p) == status
    lib.ftrainPatternDestroy(p)


def test_two_producers_and_cycles_are_rejected(lib):
    p = new_pattern(lib)
    ids = add_tensors(lib, p, 7)
    op = c.RoleId()
    lib.ftrainPatternAddGemm(p, ctypes.byref(op), ids[0], ids[1], ids[2], ids[3], ids[4], ids[5])
    lib.ftrainPatternAddGemm(p, ctypes.byref(op), ids[1], ids[0], ids[2], ids[3], ids[4], ids[6])
    assert ops_status(lib, p) == c.INVALID_ARGUMENT
    assert b"already has a producer" in lib.ftrainGetLastMessage()
    lib.ftrainPatternDestroy(p)
    # a -> d1 via op0, d1 -> a via op1: a dependency cycle.
    p = new_pattern(lib)
    ids = add_tensors(lib, p, 8)
    lib.ftrainPatternAddGemm(p, ctypes.byref(op), ids[0], ids[1], ids[2], ids[3], ids[4], ids[5])
    lib.ftrainPatternAddGemm(p, ctypes.byref(op), ids[3], ids[6], ids[7], ids[0], ids[4], ids[5])
    assert ops_status(lib, p) == c.INVALID_ARGUMENT
    assert b"cycle" in lib.ftrainGetLastMessage()
    lib.ftrainPatternDestroy(p)


def test_unsupported_patterns(lib):
    op = c.RoleId()
    # Extra isolated operand.
    p = new_pattern(lib)
    ids = add_tensors(lib, p, 7)
    lib.ftrainPatternAddGemm(p, ctypes.byref(op), *ids[:6])
    assert ops_status(lib, p) == c.UNSUPPORTED
    lib.ftrainPatternDestroy(p)
    # Two chained Gemms.
    p = new_pattern(lib)
    ids = add_tensors(lib, p, 9)
    lib.ftrainPatternAddGemm(p, ctypes.byref(op), ids[0], ids[1], ids[2], ids[3], ids[4], ids[5])
    lib.ftrainPatternAddGemm(p, ctypes.byref(op), ids[3], ids[6], ids[7], ids[8], ids[4], ids[5])
    assert ops_status(lib, p) == c.UNSUPPORTED
    lib.ftrainPatternDestroy(p)
    # Empty pattern: nothing matches.  (A grouped Gemm pattern has an engine
    # here; the reference declares the kind without one.)
    p = new_pattern(lib)
    assert ops_status(lib, p) == c.UNSUPPORTED
    g = []
    for _ in range(4):
        r = c.RoleId()
        lib.ftrainPatternAddGroupedTensor(p, ctypes.byref(r))
        g.append(r)
    al, be = add_tensors(lib, p, 2)
    assert lib.ftrainPatternAddGroupedABCDGemm(p, ctypes.byref(op), g[0], g[1], g[2], g[3], al, be) == c.SUCCESS
    assert ops_status(lib, p) == c.SUCCESS
    lib.ftrainPatternDestroy(p)
    # A TensorList in a Gemm port.
    p = new_pattern(lib)
    ids = add_tensors(lib, p, 5)
    tl = c.RoleId()
    lib.ftrainPatternAddTensorList(p, ctypes.byref(tl))
    lib.ftrainPatternAddGemm(p, ctypes.byref(op), tl, ids[0], ids[1], ids[2], ids[3], ids[4])
    assert ops_status(lib, p) == c.UNSUPPORTED
    lib.ftrainPatternDestroy(p)


def test_ops_outlives_pattern(lib):
    ops = c.GemmOps(order=("beta", "d", "a", "alpha", "c", "b"))
    args = c.Args.__new__(c.Args)  # noqa: F841 (constructed below through ops)
    al, be = c.HostScalar(1.0), c.HostScalar(0.0)
    a = ops.args(c.View(FAKE, [4, 4]), c.View(FAKE, [4, 4]), c.View(None, [4, 4]), c.View(FAKE, [4, 4]), al.view,
                 be.view)
    a.close()
    ops.close()


# ------------------------------------------------------------------ Args / StorageView


@pytest.fixture
def gemm_ops():
    ops = c.GemmOps()
    yield ops
    ops.close()


def args_handle(lib, ops):
    h = ctypes.c_void_p()
    c.check(lib.ftrainArgsCreate(ctypes.byref(h), ops.ops), l=lib)
    return h


@pytest.mark.parametrize("view,why", [
    (c.View(FAKE, [2, 2], numeric_type=0), "numeric_type"),
    (c.View(FAKE, [2, 2], numeric_type=c.NUMERIC_TYPE_COUNT), "numeric_type"),
    (c.View(FAKE, [2, 2], index_type=c.INDEX_TYPE_COUNT), "index_type"),
    (c.View(None, []), "scalar"),
    (c.View(FAKE, [2, -1]), "non-negative"),
    (c.View(FAKE, [2, 2], index_type=c.INDEX_INVALID), "strides"),
    (c.View(FAKE, [2, 2], strides=[2, 1]), "strides must be null"),
])
def test_storage_view_validation(lib, gemm_ops, view, why):
    h = args_handle(lib, gemm_ops)
    assert lib.ftrainArgsSetTensor(h, gemm_ops.ids["a"], view.sv) == c.INVALID_ARGUMENT
    assert why.encode() in lib.ftrainGetLastMessage()
    lib.ftrainArgsDestroy(h)


@pytest.mark.parametrize("make", [
    # Zero-length dimension (reference storage_view_test.cpp:101-109).
    lambda: c.View(None, [2, 0, 4]),
    # Semantically odd strides are stored without validation (:111-120).
    lambda: c.View(None, [2, 4], index_type=c.INDEX_INVALID, strides=[0, -1]),
    # Highest defined numeric and index types (:122-133).
    lambda: c.View(None, [4], numeric_type=c.NUMERIC_TYPE_COUNT - 1, index_type=c.INDEX_TYPE_COUNT - 1),
])
def test_storage_view_acceptances(lib, gemm_ops, make):
    view = make()
    h = args_handle(lib, gemm_ops)
    assert lib.ftrainArgsSetTensor(h, gemm_ops.ids["a"], view.sv) == c.SUCCESS, lib.ftrainGetLastMessage()
    lib.ftrainArgsDestroy(h)


def test_rank_zero_with_non_null_metadata_is_a_scalar(lib, gemm_ops):
    # Non-null dims and strides with num_dims 0 describe a scalar (reference
    # storage_view_test.cpp:87-99): accepted for alpha.
    value = ctypes.c_float(1.0)
    dims, strides = (ctypes.c_int64 * 1)(17), (ctypes.c_int64 * 1)(19)
    sv = c.StorageView(ctypes.addressof(value), ctypes.cast(dims, ctypes.POINTER(ctypes.c_int64)),
                       ctypes.cast(strides, ctypes.POINTER(ctypes.c_int64)), 0, c.FP32, c.INDEX_INVALID, True)
    h = args_handle(lib, gemm_ops)
    assert lib.ftrainArgsSetTensor(h, gemm_ops.ids["alpha"], sv) == c.SUCCESS, lib.ftrainGetLastMessage()
    lib.ftrainArgsDestroy(h)


def test_failed_set_keeps_the_previous_operand(tlib, tops):
    # A Set that fails validation leaves the operand already bound in place
    # (reference runtime_api_test.cpp:587-628 checks the same for operation
    # attributes): the Plan is built from the earlier, valid views.
    h = ctypes.c_void_p()
    c.check(tlib.ftrainArgsCreate(ctypes.byref(h), tops.ops), l=tlib)
    al, be = c.HostScalar(1.0), c.HostScalar(0.0)
    views = {"a": V([64, 32]), "b": V([32, 48]), "c": V([64, 48], None), "d": V([64, 48]),
             "alpha": al.view, "beta": be.view}
    for role, v in views.items():
        c.check(tlib.ftrainArgsSetTensor(h, tops.ids[role], v.sv), l=tlib)
    assert tlib.ftrainArgsSetTensor(h, tops.ids["a"], V([64, -1]).sv) == c.INVALID_ARGUMENT
    assert tlib.ftrainArgsSetGemm(h, tops.gemm_id, c.NUMERIC_TYPE_COUNT) == c.INVALID_ARGUMENT
    c.check(tlib.ftrainArgsSetGemm(h, tops.gemm_id, c.FP32), l=tlib)
    p = ctypes.c_void_p()
    assert tlib.ftrainTestingPlanCreateOnDevice(ctypes.byref(p), h, 0) == c.SUCCESS, c.last_message(tlib)
    tlib.ftrainPlanDestroy(p)
    tlib.ftrainArgsDestroy(h)


def test_storage_view_null_dims_for_nonscalar(lib, gemm_ops):
    h = args_handle(lib, gemm_ops)
    sv = c.StorageView(FAKE, None, None, 2, c.FP32, c.INDEX_CONTINUOUS, False)
    assert lib.ftrainArgsSetTensor(h, gemm_ops.ids["a"], sv) == c.INVALID_ARGUMENT
    lib.ftrainArgsDestroy(h)


def test_args_role_checks(lib, gemm_ops):
    h = args_handle(lib, gemm_ops)
    v = c.View(FAKE, [2, 2])
    assert lib.ftrainArgsSetTensor(h, c.RoleId(6), v.sv) == c.INVALID_ARGUMENT          # out of range
    assert lib.ftrainArgsSetTensorList(h, gemm_ops.ids["a"], ctypes.byref(v.sv), 1) == c.INVALID_ARGUMENT
    assert b"storage family" in lib.ftrainGetLastMessage()
    assert lib.ftrainArgsSetTensorList(h, gemm_ops.ids["a"], None, 3) == c.INVALID_ARGUMENT
    assert lib.ftrainArgsSetGemm(h, gemm_ops.gemm_id, 0) == c.INVALID_ARGUMENT
    assert lib.ftrainArgsSetGemm(h, gemm_ops.gemm_id, c.NUMERIC_TYPE_COUNT) == c.INVALID_ARGUMENT
    assert lib.ftrainArgsSetGemm(h, c.RoleId(1), c.FP32) == c.INVALID_ARGUMENT
    assert lib.ftrainArgsSetGroupedABCDGemm(h, gemm_ops.gemm_id, c.FP32) == c.INVALID_ARGUMENT
    assert b"operation kind" in lib.ftrainGetLastMessage()
    assert lib.ftrainArgsSetGemm(h, gemm_ops.gemm_id, c.FP32) == c.SUCCESS
    lib.ftrainArgsDestroy(h)


def test_grouped_tensor_validation(lib, gemm_ops):
    h = args_handle(lib, gemm_ops)
    data = c.View(FAKE, [8, 4])
    bad_offsets = c.View(FAKE, [3])          # num_groups is 2
    ok_offsets = c.View(FAKE, [2])
    assert lib.ftrainArgsSetGroupedTensor(h, gemm_ops.ids["a"], 2, data.sv, ctypes.byref(bad_offsets.sv), None,
                                          None) == c.INVALID_ARGUMENT
    assert b"offsets" in lib.ftrainGetLastMessage()
    sizes = (c.StorageView * 2)(c.View(FAKE, [2]).sv, c.View(FAKE, [2, 1]).sv)
    assert lib.ftrainArgsSetGroupedTensor(h, gemm_ops.ids["a"], 2, data.sv, ctypes.byref(ok_offsets.sv), sizes,
                                          None) == c.INVALID_ARGUMENT
    assert b"dim_sizes" in lib.ftrainGetLastMessage()
    # A valid GroupedTensor value still cannot bind to a Tensor role.
    assert lib.ftrainArgsSetGroupedTensor(h, gemm_ops.ids["a"], 2, data.sv, ctypes.byref(ok_offsets.sv), None,
                                          None) == c.INVALID_ARGUMENT
    assert b"storage family" in lib.ftrainGetLastMessage()
    lib.ftrainArgsDestroy(h)


# ------------------------------------------------------------------ Plan creation (device id given)


def plan_status(tlib, ops, a, b, cc, d, alpha=1.0, beta=0.0, compute=c.FP32, device=0, alpha_view=None,
                beta_view=None):
    al, be = c.HostScalar(alpha), c.HostScalar(beta)
    args = ops.args(a, b, cc, d, alpha_view or al.view, beta_view or be.view, compute_type=compute)
    h = ctypes.c_void_p()
    st = tlib.ftrainTestingPlanCreateOnDevice(ctypes.byref(h), args.handle, device)
    msg = c.last_message(tlib)
    plan = c.Plan(h, tlib) if st == c.SUCCESS else None
    args.close()
    return st, msg, plan


@pytest.fixture(scope="module")
def tops(tlib):
    return c.GemmOps(order=("d", "beta", "alpha", "c", "b", "a"), l=tlib)


def V(dims, mem=FAKE, **kw):
    return c.View(mem, dims, **kw)


def test_incomplete_args(tlib, tops):
    h = ctypes.c_void_p()
    tlib.ftrainArgsCreate(ctypes.byref(h), tops.ops)
    p = ctypes.c_void_p()
    assert tlib.ftrainTestingPlanCreateOnDevice(ctypes.byref(p), h, 0) == c.INVALID_ARGUMENT
    assert b"unset" in tlib.ftrainGetLastMessage()
    tlib.ftrainArgsDestroy(h)


def test_plan_success_and_queries(tlib, tops):
    st, msg, plan = plan_status(tlib, tops, V([64, 32]), V([32, 48]), V([64, 48]), V([64, 48]))
    assert st == c.SUCCESS, msg
    names = plan.names()
    assert len(names) >= 1 and len(set(names)) == len(names)
    assert all(plan.workspace_bytes(i) == 0 for i in range(len(names)))
    s = ctypes.c_char_p()
    assert tlib.ftrainPlanGetPrimitiveName(plan.handle, len(names), ctypes.byref(s)) == c.INVALID_ARGUMENT
    n = ctypes.c_uint64()
    assert tlib.ftrainPlanGetPrimitiveRequiredWorkspaceBytes(plan.handle, 99, ctypes.byref(n)) == c.INVALID_ARGUMENT
    assert "Fp32Gemm" in names  # the universal kernel applies to every valid fp32 problem
    plan.close()


@pytest.mark.parametrize("a,b,cc,d", [
    (V([6]), V([2, 4]), V([3, 4]), V([3, 4])),
    (V([3, 2]), V([3, 4]), V([3, 4]), V([3, 4])),
    (V([3, 2]), V([2, 4]), V([3, 4]), V([4, 3])),
    (V([3, 2]), V([2, 4]), V([3, 5]), V([3, 4])),
    (V([3, 2], host=True), V([2, 4]), V([3, 4]), V([3, 4])),
])
def test_invalid_shapes_and_placement(tlib, tops, a, b, cc, d):
    st, msg, _ = plan_status(tlib, tops, a, b, cc, d)
    assert st == c.INVALID_ARGUMENT, msg


def test_scalar_rules(tlib, tops):
    x = ctypes.c_float(1.0)
    st, msg, _ = plan_status(tlib, tops, V([3, 2]), V([2, 4]), V([3, 4]), V([3, 4]),
                             alpha_view=c.View(ctypes.addressof(x), [1], host=True))
    assert st == c.INVALID_ARGUMENT and "scalar" in msg
    st, msg, _ = plan_status(tlib, tops, V([3, 2]), V([2, 4]), V([3, 4]), V([3, 4]),
                             alpha_view=c.View(FAKE, []))  # device scalar
    assert st == c.INVALID_ARGUMENT and "host" in msg


def test_overflow(tlib, tops):
    big = (1 << 63) - 1
    st, msg, _ = plan_status(tlib, tops, V([big, big], None), V([big, big], None), V([big, big], None),
                             V([big, big], None))
    assert st == c.OVERFLOW, msg


@pytest.mark.parametrize("kw,why", [
    (dict(a=V([3, 2], numeric_type=c.FP16)), "an operand is not fp32"),
    (dict(b=V([2, 4], numeric_type=c.FP64)), "an operand is not fp32"),
    # The reference rejects every explicit-stride view (gemm_api_test.cpp:279-287); strides that only
    # restate the continuous layout are still rejected here, other layouts are accepted below.
    (dict(a=V([3, 2], index_type=c.INDEX_INVALID, strides=[2, 1])), "restate the continuous layout"),
    (dict(a=V([3, 2], index_type=c.INDEX_GROUPED_CONTINUOUS)), "continuously indexed"),
    (dict(a=V([3, 2], index_type=c.INDEX_INVALID, strides=[-2, 1])), "stride is negative"),
    (dict(a=V([3, 2], index_type=c.INDEX_INVALID, strides=[4, 2])), "unit stride"),
    (dict(a=V([3, 2], index_type=c.INDEX_INVALID, strides=[1, 2])), "unit stride"),  # columns overlap
    (dict(d=V([3, 4], index_type=c.INDEX_INVALID, strides=[1, 3])), "one orientation"),
    (dict(compute=c.FP64), "compute type is not fp32"),
    (dict(a=V([3, 2], None)), "required operand address is null"),
    (dict(d=V([3, 4], None)), "required operand address is null"),
    (dict(a=V([3, 2], FAKE + 2)), "not float-aligned"),
])
def test_unsupported_reasons_name_every_primitive(tlib, tops, kw, why):
    args = dict(a=V([3, 2]), b=V([2, 4]), cc=V([3, 4]), d=V([3, 4]))
    args.update({k: v for k, v in kw.items() if k != "compute"})
    st, msg, _ = plan_status(tlib, tops, args["a"], args["b"], args["cc"], args["d"],
                             compute=kw.get("compute", c.FP32))
    assert st == c.UNSUPPORTED, msg
    assert why in msg
    assert len(msg) <= 2047
    # Rejections are grouped by reason ("A, B: reason; C: other"); every
    # variant is named unless the message reached the 2047-character cap.
    for v in range(tlib.ftrainTestingVariantCount()):
        name = tlib.ftrainTestingVariantName(v).decode()
        assert name in msg or len(msg) == 2047, (name, msg)
    assert msg.count(": " + why) <= 1 or why == "", msg


@pytest.mark.parametrize("formatted", [True, False])
@pytest.mark.parametrize("length,kept", [(10, 10), (2046, 2046), (2047, 2047), (2048, 2047), (10000, 2047)])
def test_last_message_holds_at_most_2047_characters(tlib, formatted, length, kept):
    """Reference error.hpp:17,52: 2048 bytes of storage, terminator included."""
    tlib.ftrainTestingFailWithLength.restype = ctypes.c_int
    tlib.ftrainTestingFailWithLength.argtypes = [ctypes.c_int, ctypes.c_size_t, ctypes.c_bool]
    st = tlib.ftrainTestingFailWithLength(c.UNSUPPORTED, length, formatted)
    assert st == c.UNSUPPORTED
    assert tlib.ftrainGetLastStatus() == c.UNSUPPORTED
    msg = ctypes.string_at(tlib.ftrainGetLastMessage())
    assert msg == b"x" * kept


def test_failure_with_success_status_reports_internal_error(tlib):
    tlib.ftrainTestingFailWithLength.restype = ctypes.c_int
    tlib.ftrainTestingFailWithLength.argtypes = [ctypes.c_int, ctypes.c_size_t, ctypes.c_bool]
    st = tlib.ftrainTestingFailWithLength(c.SUCCESS, 5, False)
    assert st == c.INTERNAL_ERROR
    assert b"success status" in ctypes.string_at(tlib.ftrainGetLastMessage())


def S(dims, strides, mem=FAKE):
    """Explicit-stride device view."""
    return c.View(mem, dims, index_type=c.INDEX_INVALID, strides=strides)


@pytest.mark.parametrize("a,b,cc,d", [
    (S([64, 32], [1, 64]), V([32, 48]), V([64, 48]), V([64, 48])),          # a column-major
    (V([64, 32]), S([32, 48], [1, 32]), V([64, 48]), V([64, 48])),          # b column-major
    (S([64, 32], [1, 64]), S([32, 48], [1, 32]), V([64, 48]), V([64, 48])),  # both
    (S([64, 32], [40, 1]), S([32, 48], [52, 1]), S([64, 48], [56, 1]), S([64, 48], [60, 1])),  # padded rows
    (V([64, 32]), V([32, 48]), S([64, 48], [1, 64]), S([64, 48], [1, 68])),  # c, d column-major
    (V([64, 32]), V([32, 48]), V([64, 48], None), S([64, 48], [1, 64])),     # d column-major, no c
])
def test_strided_layouts_get_plans(tlib, tops, a, b, cc, d):
    st, msg, plan = plan_status(tlib, tops, a, b, cc, d)
    assert st == c.SUCCESS, msg
    names = plan.names()
    assert "Fp32Gemm" in names
    # Variants built for row-major a and b only drop out when an operand is column-major.
    if any(v.sv.index_type == c.INDEX_INVALID and v.sv.strides[0] == 1 for v in (a, b, d)):
        assert "Fp32MfmaGemm_256x256" not in names
    plan.close()


def test_strided_alignment_rules(tlib, tops):
    # Leading dimension not a multiple of 4: only per-element variants remain.
    st, msg, plan = plan_status(tlib, tops, S([64, 32], [1, 65]), V([32, 48]), V([64, 48]), V([64, 48]))
    assert st == c.SUCCESS, msg
    assert all("Unaligned" in n or n == "Fp32Gemm" for n in plan.names()), plan.names()
    plan.close()
    # Column-major a with m % 4 != 0 cannot use 128-bit loads along m.
    st, msg, plan = plan_status(tlib, tops, S([63, 32], [1, 64]), V([32, 48]), V([63, 48]), V([63, 48]))
    assert st == c.SUCCESS, msg
    assert all("Unaligned" in n or n == "Fp32Gemm" for n in plan.names()), plan.names()
    plan.close()


def test_split_k_primitives_report_their_partial_bytes(tlib, tops):
    """Without Plan preparation (the host hook skips it) every split-k
    Primitive states its workspace: 16 KiB of arrival counters, then a whole
    number (at least two) of m x n fp32 partial slices (the _SplitK kernels)
    or of 64 x 64 partial tiles per output tile (the _DeepK kernel), within
    the 256 MiB cap.  Whole-k Primitives need none."""
    m, n, k = 64, 4096, 4096
    st, msg, plan = plan_status(tlib, tops, V([m, k]), V([k, n]), V([m, n], None), V([m, n]))
    assert st == c.SUCCESS, msg
    split = 0
    for i, name in enumerate(plan.names()):
        w = plan.workspace_bytes(i)
        unit = m * n * 4 if name.endswith("SplitK") else 4096 * 4 * ((m + 63) // 64) * ((n + 63) // 64)
        if name.endswith(("SplitK", "DeepK")):
            split += 1
            assert (w - 16384) % unit == 0 and 2 <= (w - 16384) // unit and w <= 256 << 20, (name, w)
        else:
            assert w == 0, (name, w)
    assert split >= 3 and plan.names()[0].endswith(("SplitK", "DeepK")), plan.names()
    plan.close()


def test_empty_output_needs_no_storage(tlib, tops):
    st, msg, plan = plan_status(tlib, tops, V([0, 2], None), V([2, 4], None), V([0, 4], None), V([0, 4], None))
    assert st == c.SUCCESS, msg
    assert plan.workspace_bytes(0) == 0


def test_zero_depth_needs_no_a_or_b(tlib, tops):
    st, msg, plan = plan_status(tlib, tops, V([3, 0], None), V([0, 4], None), V([3, 4]), V([3, 4]))
    assert st == c.SUCCESS, msg
    assert not any(n.startswith("Fp32MfmaGemm") and n.endswith("SplitK") for n in plan.names())


# ------------------------------------------------------------------ Finder choices


def rank(tlib, m, n, k, addr=FAKE, with_c=False, device=0, ab_type=c.FP32):
    views = (c.StorageView * 6)()
    keep = [V([m, k], addr, numeric_type=ab_type), V([k, n], addr, numeric_type=ab_type),
            V([m, n], addr if with_c else None), V([m, n], addr)]
    al, be = c.HostScalar(1.0), c.HostScalar(0.0)
    for i, v in enumerate(keep + [al.view, be.view]):
        views[i] = v.sv
    buf = ctypes.create_string_buffer(4096)
    st = tlib.ftrainTestingRankGemm(views, c.FP32, device, buf, 4096)
    assert st == c.SUCCESS, c.last_message(tlib)
    return buf.value.decode().split(",")


def test_finder_choices_for_the_baseline_configs(tlib):
    # Best of 3 interleaved passes over every applicable Primitive, MI355X, N(0,1) inputs (us):
    # 8192^3: the DMA-staged 128x128 tile 7143, DMA 256x256 ~7200, the register-staged 16x16
    # 256x256 7694.  MLP fwd / dgrad: DMA 128x128 12547 / 12474 (register-staged 13529 / 13426).
    assert rank(tlib, 8192, 8192, 8192)[0] in ("Fp32Mfma16Gemm_128x128_Dma", "Fp32Mfma16Gemm_256x256_Dma")
    assert rank(tlib, 16384, 14336, 4096)[0] in ("Fp32Mfma16Gemm_128x128_Dma", "Fp32Mfma16Gemm_256x256_Dma")
    assert rank(tlib, 16384, 4096, 14336)[0].startswith("Fp32Mfma16Gemm_")
    # 6144^3: DMA 128x128 3026 (two workgroups per CU: 2.25 tiles per CU of the 256x256 tiles
    # leave a ragged last round), the 32x32 128x128 tile 3375.
    assert rank(tlib, 6144, 6144, 6144)[0] == "Fp32Mfma16Gemm_128x128_Dma"
    assert rank(tlib, 4096, 4096, 4096, with_c=True)[0].startswith("Fp32Mfma16Gemm_")
    # 2048^3: DMA 128x64 117.4, 64x128 117.6, 128x128 122.0, its split-k form 127.1, the
    # register-staged 256x64 139.1.
    assert rank(tlib, 2048, 2048, 2048)[0] in ("Fp32Mfma16Gemm_128x64_Dma", "Fp32Mfma16Gemm_64x128_Dma",
                                               "Fp32Mfma16Gemm_128x128_Dma")
    # 1024^3: DMA 64x128 split-k 25.7, the deep-k tile unsplit 26.7, DMA 128x64 split-k 27.9.
    assert rank(tlib, 1024, 1024, 1024)[0] in ("Fp32Mfma16Gemm_64x64_DeepK", "Fp32Mfma16Gemm_64x128_Dma_SplitK",
                                               "Fp32Mfma16Gemm_64x64_Dma_SplitK")
    # GEMV: the one-pass kernel (37.8 us) against split-k plus its reduction (47.6 us).
    assert rank(tlib, 1, 8192, 8192)[0] == "Fp32Gemv"
    # It also wins with 128 (1x4096x8192: 24.8 against 39.2 us) and 64 workgroups of 16 waves
    # (2x2048x4096: 11.0 against 13.1 for the 64x128 DMA split-k tile), and with fewer workgroups
    # over a short k (1x1024x4096: 6.7 against 9.5 for the 64x64 DMA split-k tile).  The split-k
    # skinny kernel lost everywhere it was measured: 1x1024x8192 19.1 against 13.1 for the 64x128
    # DMA split-k tile, 8x1024x8192 40.1 against 13.4.
    assert rank(tlib, 1, 4096, 8192)[0] == "Fp32Gemv"
    assert rank(tlib, 2, 2048, 4096)[0] == "Fp32Gemv"
    assert rank(tlib, 1, 1024, 4096)[0] == "Fp32Gemv"
    assert rank(tlib, 1, 1024, 8192)[0].endswith("_Dma_SplitK")
    assert rank(tlib, 8, 1024, 8192)[0].endswith("_Dma_SplitK")
    # Skinny and deep k (model-chosen split counts): 64x4096x4096: DMA 64x64 split-k 26.7, 64x128
    # 27.0, 64x256 28.6, deep-k 29.0; 4096x64x4096: DMA 64x64 split-k 25.6, 128x64 26.7, 256x64
    # 29.2; 256x256x65536: DMA 128x64 split-k 66.2, 64x128 66.4, 64x64 68.1, 256x64 75.2;
    # 64x1024x16384: DMA 64x64 split-k 25.4, 64x128 26.9, 64x256 28.5.
    small = ("Fp32Mfma16Gemm_64x64_Dma_SplitK", "Fp32Mfma16Gemm_64x128_Dma_SplitK", "Fp32Mfma16Gemm_128x64_Dma_SplitK")
    assert rank(tlib, 256, 256, 65536)[0] in small
    assert rank(tlib, 64, 1024, 16384)[0] in small
    assert rank(tlib, 64, 4096, 4096)[0] in small
    assert rank(tlib, 4096, 64, 4096)[0] in small
    # Odd sizes: no 128-bit variant applies.
    odd = rank(tlib, 127, 97, 33)
    assert odd and all(("Unaligned" in n) or n == "Fp32Gemm" for n in odd)


def test_finder_choices_for_16_bit_skinny_m(tlib):
    # bf16, MI355X (us): the one-pass kernel against the 64x128 DMA split-k tile: one row 23.9 / 4.6 /
    # 3.9 against 25.4 / 7.3 / 7.3 (8192^2, 2048^2, 1x4096x1024), two rows 26.2 / 5.8 against 25.8 /
    # 7.2; four rows 31.0 / 17.9 against 26.5 / 9.2 (8192^2, 4096^2), so it takes at most two rows.
    # 64 workgroups (4096 columns) are bound by what each CU loads: 1x4096x4096 ties (9.0 against 9.1).
    for t in (c.BF16, c.FP16):
        name = "Bf16Gemv" if t == c.BF16 else "Fp16Gemv"
        tile = "Bf16MfmaGemm_64x128_Dma_SplitK" if t == c.BF16 else "Fp16MfmaGemm_64x128_Dma_SplitK"
        assert rank(tlib, 1, 8192, 8192, ab_type=t)[0] == name
        assert rank(tlib, 1, 2048, 2048, ab_type=t)[0] == name
        assert rank(tlib, 2, 2048, 2048, ab_type=t)[0] == name
        assert rank(tlib, 1, 4096, 1024, ab_type=t)[0] == name
        assert rank(tlib, 1, 4096, 4096, ab_type=t)[0] in (name, tile)
        assert name not in rank(tlib, 3, 8192, 8192, ab_type=t)
        assert rank(tlib, 4, 4096, 4096, ab_type=t)[0] == tile


def test_finder_choices_for_16_bit_tiles(tlib):
    # bf16, MI355X, every applicable Primitive timed (us): the Finder's pick was the fastest on each
    # of these.  Small and mid-size squares: the 128x128 DMA tile (2048^3 25.3 against 256x256 DMA
    # 39.1); large ones: the 256x256 DMA tile (8192^3 871 against 128x128 DMA 906); deep k: the
    # 128x128 DMA split-k tile (256x256x65536 21.2 against the register-staged split-k 29.3).
    assert rank(tlib, 2048, 2048, 2048, ab_type=c.BF16)[0] == "Bf16MfmaGemm_128x128_Dma"
    # Few whole-k workgroups, each bound by its own CU's load rate: 128x4096x1024 9.3 us against 13.2
    # for the split tile, 4096x128x1024 9.5 against 13.4, 128x256x512 6.5 against 10.7 for the 64x64
    # unaligned tile.
    for shape in ((128, 4096, 1024), (4096, 128, 1024), (128, 256, 512)):
        assert rank(tlib, *shape, ab_type=c.BF16)[0] == "Bf16MfmaGemm_128x128_Dma", shape
    assert rank(tlib, 8192, 8192, 8192, ab_type=c.BF16)[0] == "Bf16MfmaGemm_256x256_Dma"
    assert rank(tlib, 16384, 14336, 4096, ab_type=c.BF16)[0] == "Bf16MfmaGemm_256x256_Dma"
    for shape in ((256, 256, 65536), (384, 4096, 4096), (1536, 1536, 8192)):
        assert rank(tlib, *shape, ab_type=c.BF16)[0] == "Bf16MfmaGemm_128x128_Dma_SplitK", shape
    # One tile row: the 64x128 DMA split tile, at the split count measured fastest (after a warm
    # clock, forced split counts, us): 64x4096x4096 12.7 at 8 splits (128x128 split tile 13.5),
    # 64x4096x14336 23.8 at 8 (25.4), 64x14336x4096 23.7 at 2 (26.3 at 4; 224 workgroups, 85% of the
    # CUs, already stream at the full rate), 32x14336x4096 22.8 at 2 (24.3 at 4); 4 splits of
    # 64x4096x14336 (128 workgroups) took 36.3.
    tile64 = "Bf16MfmaGemm_64x128_Dma_SplitK"
    names = {tlib.ftrainTestingVariantName(i).decode(): i for i in range(tlib.ftrainTestingVariantCount())}
    for shape, splits in (((64, 4096, 4096), 8), ((64, 4096, 14336), 8), ((64, 14336, 4096), 2),
                          ((32, 14336, 4096), 2)):
        assert rank(tlib, *shape, ab_type=c.BF16)[0] == tile64, shape
        assert tlib.ftrainTestingChooseSplits(names[tile64], *shape, 256) == splits, shape
    # k not a multiple of 64: the DMA tiles stage the partial last stage and still lead (bf16, us:
    # 8192x8192x8200 819 against 944 for the register-staged 256x256 tile, 16384x14336x4104 1491
    # against 1764); a k that is not a multiple of 8 (row-major a) leaves only the per-element tile.
    assert rank(tlib, 8192, 8192, 8200, ab_type=c.BF16)[0] == "Bf16MfmaGemm_256x256_Dma"
    assert rank(tlib, 16384, 14336, 4104, ab_type=c.BF16)[0] == "Bf16MfmaGemm_256x256_Dma"
    assert rank(tlib, 4096, 4096, 4100, ab_type=c.BF16) == ["Bf16MfmaGemm_64x64_Unaligned"]
    # Taller problems keep the 128-row tiles: the 64-row one does not apply above m = 64.
    assert tile64 not in rank(tlib, 65, 4096, 4096, ab_type=c.BF16)
    assert "Fp16MfmaGemm_64x128_Dma_SplitK" == rank(tlib, 64, 4096, 4096, ab_type=c.FP16)[0]


def test_finder_respects_alignment_and_row_limits(tlib):
    names = rank(tlib, 512, 512, 512, addr=FAKE + 4)
    assert names and all(("Unaligned" in n) or n == "Fp32Gemm" for n in names)
    assert not any(n.startswith("Fp32Gemv") for n in rank(tlib, 9, 8192, 8192))
    assert "Fp32Gemv_SplitK" in rank(tlib, 8, 8192, 8192)
    assert "Fp32Gemv" in rank(tlib, 8, 8192, 8192)


def test_plan_order_matches_finder_rank(tlib, tops):
    st, msg, plan = plan_status(tlib, tops, V([1, 8192]), V([8192, 8192]), V([1, 8192], None), V([1, 8192]))
    assert st == c.SUCCESS, msg
    assert plan.names() == rank(tlib, 1, 8192, 8192)


def test_cost_model_is_monotone_in_work(tlib):
    for v in range(tlib.ftrainTestingVariantCount()):
        small = tlib.ftrainTestingEstimateMicros(v, 1024, 1024, 1024, False, 256)
        large = tlib.ftrainTestingEstimateMicros(v, 4096, 4096, 4096, False, 256)
        if small != float("inf"):
            assert large >= small, tlib.ftrainTestingVariantName(v)


def test_split_counts(tlib):
    names = {tlib.ftrainTestingVariantName(v).decode(): v for v in range(tlib.ftrainTestingVariantCount())}
    s = tlib.ftrainTestingChooseSplits(names["Fp32MfmaGemm_128x128_SplitK"], 256, 256, 65536, 256)
    assert 2 <= s <= 65536 // 256
    assert tlib.ftrainTestingChooseSplits(names["Fp32MfmaGemm_128x128_SplitK"], 256, 256, 300, 256) == 0
    assert tlib.ftrainTestingChooseSplits(names["Fp32MfmaGemm_128x128"], 256, 256, 65536, 256) == 1
    assert tlib.ftrainTestingChooseSplits(names["Fp32Gemv_SplitK"], 1, 64, 16, 256) == 1


# ------------------------------------------------------------------ environment filters


def run_with_env(env: dict, code: str) -> str:
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    full = dict(os.environ, **env)
    prog = ("import sys; sys.path[:0]=[%r, %r]\n" % (os.path.join(repo, "flash-train_amd"), repo)) + code
    out = subprocess.run([sys.executable, "-c", prog], env=full, capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    return out.stdout.strip()


PLAN_NAMES = """
import ctypes
from flash_train import capi as c
t = c.testing_lib()
ops = c.GemmOps(l=t)
al, be = c.HostScalar(1.0), c.HostScalar(0.0)
F = 0x7F0000000000
args = ops.args(c.View(F, [2048, 2048]), c.View(F, [2048, 2048]), c.View(None, [2048, 2048]),
                c.View(F, [2048, 2048]), al.view, be.view)
h = ctypes.c_void_p()
st = t.ftrainTestingPlanCreateOnDevice(ctypes.byref(h), args.handle, 0)
print(",".join(c.Plan(h, t).names()) if st == 0 else "status=%d %s" % (st, c.last_message(t)))
"""


def test_env_disabled_primitive():
    names = run_with_env({"FTRAIN_DISABLED_PRIMITIVES": " Fp32MfmaGemm_256x256 ,\tFp32Gemm"}, PLAN_NAMES).split(",")
    assert "Fp32MfmaGemm_256x256" not in names and "Fp32Gemm" not in names and names


def test_env_enabled_primitives():
    names = run_with_env({"FTRAIN_ENABLED_PRIMITIVES": "Fp32Gemm,NoSuchPrimitive"}, PLAN_NAMES).split(",")
    assert names == ["Fp32Gemm"]


def test_env_all_filtered_is_unsupported():
    out = run_with_env({"FTRAIN_ENABLED_PRIMITIVES": "NoSuchPrimitive"}, PLAN_NAMES)
    assert out.startswith("status=4")


def test_env_disabled_finder_falls_back_to_registration_order():
    names = run_with_env({"FTRAIN_DISABLED_FINDERS": "ShapeCost"}, PLAN_NAMES).split(",")
    t = c.testing_lib()
    catalog = [t.ftrainTestingVariantName(v).decode() for v in range(t.ftrainTestingVariantCount())]
    assert names == [n for n in catalog if n in names]  # registration order
    assert names[-1] == "Fp32Gemm"


def test_env_disable_cache_still_selects_the_same():
    assert run_with_env({"FTRAIN_DISABLE_CACHE": "1"}, PLAN_NAMES) == run_with_env({"FTRAIN_DISABLE_CACHE": "0"},
                                                                                  PLAN_NAMES)


def test_name_list_and_switch_parsing(tlib):
    buf = ctypes.create_string_buffer(256)
    tlib.ftrainTestingParseNameList(b" a ,b,,\tc\t, a", buf, 256)
    assert buf.value == b"a|b|c"
    tlib.ftrainTestingParseNameList(None, buf, 256)
    assert buf.value == b""
    assert not tlib.ftrainTestingParseSwitch(None)
    assert not tlib.ftrainTestingParseSwitch(b" 0 ")
    assert not tlib.ftrainTestingParseSwitch(b"  ")
    assert tlib.ftrainTestingParseSwitch(b"1") and tlib.ftrainTestingParseSwitch(b" yes")


# ------------------------------------------------------------------ selection cache


def arr(xs):
    return (ctypes.c_uint64 * max(len(xs), 1))(*xs), len(xs)


def cache_publish(t, cache, ct, pt, pos):
    a, na = arr(ct)
    b, nb = arr(pt)
    p, npos = arr(pos)
    return t.ftrainTestingCachePublish(cache, a, na, b, nb, p, npos)


def cache_find(t, cache, ct, pt):
    a, na = arr(ct)
    b, nb = arr(pt)
    out = (ctypes.c_uint64 * 64)()
    n = t.ftrainTestingCacheFind(cache, a, na, b, nb, out, 64)
    return None if n < 0 else list(out[:n])


def test_cache_publish_once_and_key_separation(tlib):
    cache = tlib.ftrainTestingCacheCreate(1000, 4)
    assert cache_find(tlib, cache, [0], [1, 2, 3]) is None
    assert cache_publish(tlib, cache, [0], [1, 2, 3], [4, 2]) == c.SUCCESS
    assert cache_publish(tlib, cache, [0], [1, 2, 3], [9]) == c.SUCCESS  # publish-once: keeps [4, 2]
    assert cache_find(tlib, cache, [0], [1, 2, 3]) == [4, 2]
    assert cache_find(tlib, cache, [1], [1, 2, 3]) is None   # other device
    assert cache_find(tlib, cache, [0, 1], [2, 3]) is None   # token boundary moves
    assert cache_publish(tlib, cache, [0], [7], []) == c.INVALID_ARGUMENT
    assert tlib.ftrainTestingCacheSize(cache) == 1
    tlib.ftrainTestingCacheDestroy(cache)
    assert tlib.ftrainTestingCacheCreate(0, 4) is None
    assert tlib.ftrainTestingCacheCreate(10, 0) is None


def test_cache_evicts_least_hit_batch(tlib):
    cache = tlib.ftrainTestingCacheCreate(16, 1)
    for i in range(16):
        cache_publish(tlib, cache, [0], [i], [i])
    for _ in range(3):
        for i in range(8, 16):
            assert cache_find(tlib, cache, [0], [i]) == [i]
    cache_publish(tlib, cache, [0], [100], [100])
    assert tlib.ftrainTestingCacheSize(cache) == 16 - 2 + 1  # one batch of 16/8 evicted
    assert all(cache_find(tlib, cache, [0], [i]) == [i] for i in range(8, 16))  # hot entries survive
    assert cache_find(tlib, cache, [0], [100]) == [100]
    tlib.ftrainTestingCacheDestroy(cache)


def test_cache_concurrent_publishers(tlib):
    cache = tlib.ftrainTestingCacheCreate(100000, 256)

    def work(seed):
        for i in range(500):
            cache_publish(tlib, cache, [seed % 2], [i], [seed])

    threads = [threading.Thread(target=work, args=(s,)) for s in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert tlib.ftrainTestingCacheSize(cache) == 1000
    for dev in (0, 1):
        for i in (0, 250, 499):
            assert cache_find(tlib, cache, [dev], [i])[0] % 2 == dev
    tlib.ftrainTestingCacheDestroy(cache)


def test_concurrent_plan_creation_agrees(tlib, tops):
    results = []

    def work():
        st, msg, plan = plan_status(tlib, tops, V([1000, 1000]), V([1000, 1000]), V([1000, 1000], None),
                                    V([1000, 1000]))
        results.append((st, tuple(plan.names()) if plan else msg))

    threads = [threading.Thread(target=work) for _ in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(set(results)) == 1 and results[0][0] == c.SUCCESS


def test_matrix_view_keeps_the_strides_of_a_padded_tensor():
    # A non-contiguous tensor keeps its element strides also when the caller repeats its shape (the
    # c argument of plan_for); a different shape for such a tensor is refused rather than read as
    # contiguous.
    torch = pytest.importorskip("torch")
    padded = torch.zeros(4, 10)[:, :6]
    for v in (c.matrix(padded), c.matrix(padded, [4, 6])):
        assert v.sv.index_type == c.INDEX_INVALID
        assert [v.sv.strides[i] for i in range(2)] == [10, 1]
        assert [v.sv.dims[i] for i in range(2)] == [4, 6]
    with pytest.raises(ValueError):
        c.matrix(padded, [6, 4])
    dense = c.matrix(torch.zeros(4, 6), [4, 6])
    assert dense.sv.index_type == c.INDEX_CONTINUOUS and not dense.sv.strides
