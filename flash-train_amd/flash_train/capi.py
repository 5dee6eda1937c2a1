"""ctypes mirror of the flash-train C ABI (include/flash_train/common.h, flash_train.h).

This is the binding a Python caller of the reference's C library would write
(the reference's own tests drive the same entry points from C++:
tests/api/gemm_api_test.cpp, tests/support/staged_api.hpp).  It adds thin
helpers for the Gemm Pattern and for views over torch tensors.

``torch`` is imported before the library is loaded so that both use the one
HIP runtime already in the process.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_bool, c_char_p, c_double, c_int, c_int32, c_int64, c_size_t, c_uint8, c_uint32
from ctypes import c_uint64, c_void_p
from typing import Optional, Sequence

import torch  # noqa: F401  (HIP runtime must be loaded by torch first)

_PKG = os.path.dirname(os.path.abspath(__file__))
# FTRAIN_LIBRARY_DIR points the loader at another build of the two libraries (the checking builds
# of build.py --host-sanitizer); by default they sit next to this file.
_LIB_DIR = os.environ.get("FTRAIN_LIBRARY_DIR") or _PKG
LIBRARY_PATH = os.path.join(_LIB_DIR, "libflash_train.so")
TESTING_LIBRARY_PATH = os.path.join(_LIB_DIR, "libflash_train_testing.so")

# ---- enums (common.h) ----
SUCCESS, INVALID_ARGUMENT, OUT_OF_MEMORY, OVERFLOW, UNSUPPORTED, INTERNAL_ERROR = 0, 1, 2, 3, 4, 50
STATUS_NAMES = {0: "SUCCESS", 1: "INVALID_ARGUMENT", 2: "OUT_OF_MEMORY", 3: "OVERFLOW", 4: "UNSUPPORTED",
                50: "INTERNAL_ERROR"}
FP64, INT64, UINT64, FP32, INT32, UINT32, FP16, BF16 = 1, 2, 3, 4, 5, 6, 7, 8
NUMERIC_TYPE_COUNT = 24
INDEX_INVALID, INDEX_CONTINUOUS, INDEX_SF_SWIZZLED, INDEX_GROUPED_CONTINUOUS = 0, 1, 2, 3
INDEX_TYPE_COUNT = 4
TORCH_NUMERIC_TYPES = {torch.float32: FP32, torch.bfloat16: BF16, torch.float16: FP16, torch.float64: FP64}

EXPORTED_SYMBOLS = (
    "ftrainGetLastStatus", "ftrainGetLastMessage",
    "ftrainPatternCreate", "ftrainPatternDestroy", "ftrainPatternAddTensor", "ftrainPatternAddTensorList",
    "ftrainPatternAddGroupedTensor", "ftrainPatternAddGemm", "ftrainPatternAddGroupedABCDGemm",
    "ftrainPatternAddGroupedBCDGemm", "ftrainPatternAddGroupedABGemm",
    "ftrainOpsCreate", "ftrainOpsDestroy",
    "ftrainArgsCreate", "ftrainArgsDestroy", "ftrainArgsSetTensor", "ftrainArgsSetTensorList",
    "ftrainArgsSetGroupedTensor", "ftrainArgsSetGemm", "ftrainArgsSetGroupedABCDGemm",
    "ftrainArgsSetGroupedBCDGemm", "ftrainArgsSetGroupedABGemm",
    "ftrainPlanCreate", "ftrainPlanDestroy", "ftrainPlanGetNumPrimitives", "ftrainPlanGetPrimitiveName",
    "ftrainPlanGetPrimitiveRequiredWorkspaceBytes", "ftrainPlanExecutePrimitive",
    "ftrainGemm",
)
# The reference's 29 entry points plus ftrainGemmNoAlloc, which has no
# reference counterpart (for callers that cannot allocate device memory).
REFERENCE_SYMBOLS = EXPORTED_SYMBOLS
EXPORTED_SYMBOLS = REFERENCE_SYMBOLS + ("ftrainGemmNoAlloc",)


class StorageView(ctypes.Structure):
    _fields_ = [
        ("memory", c_void_p),
        ("dims", POINTER(c_int64)),
        ("strides", POINTER(c_int64)),
        ("num_dims", c_uint8),
        ("numeric_type", c_uint8),
        ("index_type", c_uint8),
        ("is_host_memory", c_bool),
    ]


class RoleId(ctypes.Structure):
    _fields_ = [("opaque", c_uint64)]


_H = c_void_p  # opaque handle


def _declare(lib: ctypes.CDLL) -> ctypes.CDLL:
    st = c_uint8
    sigs = {
        "ftrainGetLastStatus": (st, []),
        "ftrainGetLastMessage": (c_char_p, []),
        "ftrainPatternCreate": (st, [POINTER(_H)]),
        "ftrainPatternDestroy": (st, [_H]),
        "ftrainPatternAddTensor": (st, [_H, POINTER(RoleId)]),
        "ftrainPatternAddTensorList": (st, [_H, POINTER(RoleId)]),
        "ftrainPatternAddGroupedTensor": (st, [_H, POINTER(RoleId)]),
        "ftrainPatternAddGemm": (st, [_H, POINTER(RoleId)] + [RoleId] * 6),
        "ftrainPatternAddGroupedABCDGemm": (st, [_H, POINTER(RoleId)] + [RoleId] * 6),
        "ftrainPatternAddGroupedBCDGemm": (st, [_H, POINTER(RoleId)] + [RoleId] * 6),
        "ftrainPatternAddGroupedABGemm": (st, [_H, POINTER(RoleId)] + [RoleId] * 6),
        "ftrainOpsCreate": (st, [POINTER(_H), _H]),
        "ftrainOpsDestroy": (st, [_H]),
        "ftrainArgsCreate": (st, [POINTER(_H), _H]),
        "ftrainArgsDestroy": (st, [_H]),
        "ftrainArgsSetTensor": (st, [_H, RoleId, StorageView]),
        "ftrainArgsSetTensorList": (st, [_H, RoleId, POINTER(StorageView), c_uint32]),
        "ftrainArgsSetGroupedTensor": (st, [_H, RoleId, c_uint32, StorageView, POINTER(StorageView),
                                            POINTER(StorageView), POINTER(StorageView)]),
        "ftrainArgsSetGemm": (st, [_H, RoleId, c_uint8]),
        "ftrainArgsSetGroupedABCDGemm": (st, [_H, RoleId, c_uint8]),
        "ftrainArgsSetGroupedBCDGemm": (st, [_H, RoleId, c_uint8]),
        "ftrainArgsSetGroupedABGemm": (st, [_H, RoleId, c_uint8]),
        "ftrainPlanCreate": (st, [POINTER(_H), _H]),
        "ftrainPlanDestroy": (st, [_H]),
        "ftrainPlanGetNumPrimitives": (st, [_H, POINTER(c_uint64)]),
        "ftrainPlanGetPrimitiveName": (st, [_H, c_uint64, POINTER(c_char_p)]),
        "ftrainPlanGetPrimitiveRequiredWorkspaceBytes": (st, [_H, c_uint64, POINTER(c_uint64)]),
        "ftrainPlanExecutePrimitive": (st, [_H, c_uint64, c_void_p, c_uint64, c_void_p]),
        "ftrainGemm": (st, [StorageView] * 6 + [c_uint8, c_void_p, c_uint64, c_void_p]),
        "ftrainGemmNoAlloc": (st, [StorageView] * 6 + [c_uint8, c_void_p]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def _declare_testing(lib: ctypes.CDLL) -> ctypes.CDLL:
    _declare(lib)
    st = c_uint8
    sigs = {
        "ftrainTestingPlanCreateOnDevice": (st, [POINTER(_H), _H, c_int32]),
        "ftrainTestingRankGemm": (st, [POINTER(StorageView), c_uint8, c_int32, ctypes.c_char_p, c_size_t]),
        "ftrainTestingVariantCount": (c_int, []),
        "ftrainTestingVariantName": (c_char_p, [c_int]),
        "ftrainTestingEstimateMicros": (c_double, [c_int, c_uint64, c_uint64, c_uint64, c_bool, c_int]),
        "ftrainTestingChooseSplits": (c_uint32, [c_int, c_uint64, c_uint64, c_uint64, c_int]),
        "ftrainTestingForceSplits": (None, [c_uint32]),
        "ftrainTestingConveniencePlansAlive": (ctypes.c_long, []),
        "ftrainTestingCacheCreate": (c_void_p, [c_uint64, c_uint64]),
        "ftrainTestingCacheDestroy": (None, [c_void_p]),
        "ftrainTestingCachePublish": (st, [c_void_p, POINTER(c_uint64), c_size_t, POINTER(c_uint64), c_size_t,
                                           POINTER(c_uint64), c_size_t]),
        "ftrainTestingCacheFind": (c_int64, [c_void_p, POINTER(c_uint64), c_size_t, POINTER(c_uint64), c_size_t,
                                             POINTER(c_uint64), c_size_t]),
        "ftrainTestingCacheSize": (c_uint64, [c_void_p]),
        "ftrainTestingParseNameList": (None, [c_char_p, ctypes.c_char_p, c_size_t]),
        "ftrainTestingParseSwitch": (c_bool, [c_char_p]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


_lib: Optional[ctypes.CDLL] = None
_testing: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """The product library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise RuntimeError(f"{LIBRARY_PATH} is missing; run `python flash-train_amd/build.py`")
        _lib = _declare(ctypes.CDLL(LIBRARY_PATH))
    return _lib


def testing_lib() -> ctypes.CDLL:
    """The product objects plus host-only test hooks (a separate library)."""
    global _testing
    if _testing is None:
        if not os.path.exists(TESTING_LIBRARY_PATH):
            raise RuntimeError(f"{TESTING_LIBRARY_PATH} is missing; run `python flash-train_amd/build.py`")
        _testing = _declare_testing(ctypes.CDLL(TESTING_LIBRARY_PATH))
    return _testing


class FTrainError(RuntimeError):
    def __init__(self, status: int, message: str, call: str):
        super().__init__(f"{call} -> {STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


def last_message(l: Optional[ctypes.CDLL] = None) -> str:
    return ((l or lib()).ftrainGetLastMessage() or b"").decode()


def check(status: int, call: str = "ftrain", l: Optional[ctypes.CDLL] = None) -> None:
    if status != SUCCESS:
        raise FTrainError(status, last_message(l), call)


# ---- views ----

class View:
    """Keeps the dims/strides arrays of one StorageView alive."""

    def __init__(self, memory: Optional[int], dims: Sequence[int], numeric_type: int = FP32,
                 index_type: int = INDEX_CONTINUOUS, host: bool = False,
                 strides: Optional[Sequence[int]] = None):
        self._dims = (c_int64 * max(len(dims), 1))(*dims)
        self._strides = (c_int64 * max(len(strides), 1))(*strides) if strides is not None else None
        self.sv = StorageView(
            memory or None,
            ctypes.cast(self._dims, POINTER(c_int64)) if len(dims) else None,
            ctypes.cast(self._strides, POINTER(c_int64)) if self._strides is not None else None,
            len(dims), numeric_type, index_type, host)


def matrix(t: Optional[torch.Tensor], shape: Optional[Sequence[int]] = None, **kw) -> View:
    """Device matrix view over a tensor (or a null-memory view of `shape`).

    A contiguous tensor gets FTRAIN_INDEX_TYPE_CONTINUOUS; a non-contiguous
    one (a transpose, a column slice) its explicit element strides, also when
    `shape` repeats its shape.  The numeric type follows the tensor's dtype
    unless given."""
    if t is None:
        return View(None, list(shape), **kw)
    if "numeric_type" not in kw:
        kw["numeric_type"] = TORCH_NUMERIC_TYPES.get(t.dtype, FP32)
    same_shape = shape is None or list(shape) == list(t.shape)
    if not t.is_contiguous() and same_shape and "index_type" not in kw and "strides" not in kw:
        return View(t.data_ptr(), list(t.shape), index_type=INDEX_INVALID, strides=list(t.stride()), **kw)
    if not t.is_contiguous() and not same_shape:
        raise ValueError(f"a non-contiguous tensor of shape {list(t.shape)} viewed as {list(shape)}")
    return View(t.data_ptr(), list(shape) if shape is not None else list(t.shape), **kw)


class HostScalar:
    """A host fp32 scalar and its rank-0 view (kept alive together)."""

    def __init__(self, value: float, numeric_type: int = FP32):
        self.value = ctypes.c_float(value) if numeric_type == FP32 else ctypes.c_double(value)
        self.view = View(ctypes.addressof(self.value), [], numeric_type=numeric_type, host=True)


# ---- the Gemm Pattern ----

class GemmOps:
    """Pattern -> Ops for one Gemm, roles added in a caller-chosen order."""

    ORDER = ("a", "b", "c", "alpha", "beta", "d")

    def __init__(self, order: Sequence[str] = ORDER, l: Optional[ctypes.CDLL] = None):
        self.lib = l or lib()
        self.ids = {}
        pat = _H()
        check(self.lib.ftrainPatternCreate(ctypes.byref(pat)), "ftrainPatternCreate", self.lib)
        try:
            for role in order:
                rid = RoleId()
                check(self.lib.ftrainPatternAddTensor(pat, ctypes.byref(rid)), "ftrainPatternAddTensor", self.lib)
                self.ids[role] = rid
            self.gemm_id = RoleId()
            i = self.ids
            check(self.lib.ftrainPatternAddGemm(pat, ctypes.byref(self.gemm_id), i["a"], i["b"], i["c"], i["d"],
                                                i["alpha"], i["beta"]), "ftrainPatternAddGemm", self.lib)
            self.ops = _H()
            check(self.lib.ftrainOpsCreate(ctypes.byref(self.ops), pat), "ftrainOpsCreate", self.lib)
        finally:
            self.lib.ftrainPatternDestroy(pat)

    def args(self, a: View, b: View, c: View, d: View, alpha: View, beta: View, compute_type: int = FP32) -> "Args":
        return Args(self, dict(a=a, b=b, c=c, d=d, alpha=alpha, beta=beta), compute_type)

    def close(self) -> None:
        if self.ops:
            self.lib.ftrainOpsDestroy(self.ops)
            self.ops = _H()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Args:
    def __init__(self, ops: GemmOps, views: dict, compute_type: int):
        self.lib = ops.lib
        self.views = views  # keep alive until the Plan binds them
        self.handle = _H()
        check(self.lib.ftrainArgsCreate(ctypes.byref(self.handle), ops.ops), "ftrainArgsCreate", self.lib)
        for role, v in views.items():
            check(self.lib.ftrainArgsSetTensor(self.handle, ops.ids[role], v.sv), "ftrainArgsSetTensor", self.lib)
        check(self.lib.ftrainArgsSetGemm(self.handle, ops.gemm_id, compute_type), "ftrainArgsSetGemm", self.lib)

    def plan(self) -> "Plan":
        h = _H()
        check(self.lib.ftrainPlanCreate(ctypes.byref(h), self.handle), "ftrainPlanCreate", self.lib)
        return Plan(h, self.lib)

    def close(self) -> None:
        if self.handle:
            self.lib.ftrainArgsDestroy(self.handle)
            self.handle = _H()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Plan:
    def __init__(self, handle, l: ctypes.CDLL):
        self.handle, self.lib = handle, l

    def __len__(self) -> int:
        n = c_uint64()
        check(self.lib.ftrainPlanGetNumPrimitives(self.handle, ctypes.byref(n)), "ftrainPlanGetNumPrimitives",
              self.lib)
        return n.value

    def name(self, i: int = 0) -> str:
        s = c_char_p()
        check(self.lib.ftrainPlanGetPrimitiveName(self.handle, i, ctypes.byref(s)), "ftrainPlanGetPrimitiveName",
              self.lib)
        return s.value.decode()

    def names(self) -> list:
        return [self.name(i) for i in range(len(self))]

    def workspace_bytes(self, i: int = 0) -> int:
        n = c_uint64()
        check(self.lib.ftrainPlanGetPrimitiveRequiredWorkspaceBytes(self.handle, i, ctypes.byref(n)),
              "ftrainPlanGetPrimitiveRequiredWorkspaceBytes", self.lib)
        return n.value

    def execute_status(self, i: int = 0, stream: int = 0, workspace: int = 0, workspace_bytes: int = 0) -> int:
        return self.lib.ftrainPlanExecutePrimitive(self.handle, i, workspace or None, workspace_bytes, stream or None)

    def execute(self, i: int = 0, stream: int = 0, workspace: int = 0, workspace_bytes: int = 0) -> None:
        """ftrainPlanExecutePrimitive.  With no workspace given, a Primitive that
        requires one gets a device buffer of the required size, allocated once
        per Plan through torch and kept with this object."""
        if not workspace:
            need = self.workspace_bytes(i)
            if need:
                import torch

                if getattr(self, "_ws", None) is None or self._ws.numel() < need:
                    self._ws = torch.empty(need, dtype=torch.uint8, device="cuda")
                workspace, workspace_bytes = self._ws.data_ptr(), need
        check(self.execute_status(i, stream, workspace, workspace_bytes), "ftrainPlanExecutePrimitive", self.lib)

    def close(self) -> None:
        if self.handle:
            self.lib.ftrainPlanDestroy(self.handle)
            self.handle = _H()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def gemm_status(a: View, b: View, c: View, d: View, alpha: View, beta: View, compute_type: int = FP32,
                workspace: int = 0, workspace_bytes: int = 0, stream: int = 0, l: Optional[ctypes.CDLL] = None) -> int:
    """ftrainGemm (the convenience entry point); returns the status."""
    return (l or lib()).ftrainGemm(a.sv, b.sv, c.sv, d.sv, alpha.sv, beta.sv, compute_type, workspace or None,
                                   workspace_bytes, stream or None)


def gemm_no_alloc_status(a: View, b: View, c: View, d: View, alpha: View, beta: View, compute_type: int = FP32,
                         stream: int = 0, l: Optional[ctypes.CDLL] = None) -> int:
    """ftrainGemmNoAlloc (ftrainGemm with split-k partials in the library's device scratch array)."""
    return (l or lib()).ftrainGemmNoAlloc(a.sv, b.sv, c.sv, d.sv, alpha.sv, beta.sv, compute_type, stream or None)


def plan_for(a: torch.Tensor, b: torch.Tensor, c: Optional[torch.Tensor], d: torch.Tensor, alpha: float,
             beta: float, ops: Optional[GemmOps] = None) -> Plan:
    """Creates a Plan for device tensors (c may be None: null c memory).

    The Plan binds the tensors' addresses, so the returned object keeps the
    tensors alive (a temporary such as `x.cuda()` passed here would otherwise
    be freed, and its memory handed out again, while the Plan still points
    at it)."""
    ops = ops or GemmOps()
    al, be = HostScalar(alpha), HostScalar(beta)
    m, n = d.shape
    args = ops.args(matrix(a), matrix(b), matrix(c, [m, n]), matrix(d), al.view, be.view)
    try:
        plan = args.plan()
        plan._operands = (a, b, c, d)
        return plan
    finally:
        args.close()


# ---- grouped Gemm families (GroupedABCDGemm, GroupedBCDGemm, GroupedABGemm) ----

class GroupedSpec:
    """One GroupedTensor argument: a rank-two data view and per-group host int64
    descriptors (reference common.h:397-425).  `dims` and `strides` are lists of
    (rows, cols) and (row stride, column stride) per group; `offsets` lists each
    group's first element.  Any of them may be None (absent)."""

    def __init__(self, data: View, num_groups: int, dims=None, strides=None, offsets=None):
        self.data, self.num_groups = data, num_groups
        g = num_groups

        def arr(values):
            a = (c_int64 * max(g, 1))(*values)
            return a, View(ctypes.addressof(a), [g], numeric_type=INT64, host=True)

        self._keep = []
        self.dim_views = self.stride_views = self.offset_view = None
        if dims is not None:
            cols = [arr([d[i] for d in dims]) for i in range(2)]
            self._keep += cols
            self.dim_views = (StorageView * 2)(cols[0][1].sv, cols[1][1].sv)
        if strides is not None:
            cols = [arr([s[i] for s in strides]) for i in range(2)]
            self._keep += cols
            self.stride_views = (StorageView * 2)(cols[0][1].sv, cols[1][1].sv)
        if offsets is not None:
            o = arr(list(offsets))
            self._keep.append(o)
            self.offset_view = o[1]


class GroupedOps:
    """Pattern -> Ops for one grouped Gemm: kind "abcd", "bcd" (a is a TensorList) or
    "ab" (c and d are TensorLists)."""

    def __init__(self, kind: str, l: Optional[ctypes.CDLL] = None):
        self.lib = l or lib()
        self.kind = kind
        lists = {"abcd": (), "bcd": ("a",), "ab": ("c", "d")}[kind]
        self.ids, self.kinds = {}, {}
        pat = _H()
        check(self.lib.ftrainPatternCreate(ctypes.byref(pat)), "ftrainPatternCreate", self.lib)
        try:
            for role in ("a", "b", "c", "d", "alpha", "beta"):
                rid = RoleId()
                if role in ("alpha", "beta"):
                    fn, k = self.lib.ftrainPatternAddTensor, "tensor"
                elif role in lists:
                    fn, k = self.lib.ftrainPatternAddTensorList, "list"
                else:
                    fn, k = self.lib.ftrainPatternAddGroupedTensor, "grouped"
                check(fn(pat, ctypes.byref(rid)), "ftrainPatternAdd", self.lib)
                self.ids[role], self.kinds[role] = rid, k
            self.op_id = RoleId()
            add = {"abcd": self.lib.ftrainPatternAddGroupedABCDGemm, "bcd": self.lib.ftrainPatternAddGroupedBCDGemm,
                   "ab": self.lib.ftrainPatternAddGroupedABGemm}[kind]
            i = self.ids
            check(add(pat, ctypes.byref(self.op_id), i["a"], i["b"], i["c"], i["d"], i["alpha"], i["beta"]),
                  "ftrainPatternAddGrouped*Gemm", self.lib)
            self.ops = _H()
            check(self.lib.ftrainOpsCreate(ctypes.byref(self.ops), pat), "ftrainOpsCreate", self.lib)
        finally:
            self.lib.ftrainPatternDestroy(pat)

    def args(self, compute_type: int = FP32, **values) -> "GroupedArgs":
        return GroupedArgs(self, values, compute_type)

    def close(self) -> None:
        if self.ops:
            self.lib.ftrainOpsDestroy(self.ops)
            self.ops = _H()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GroupedArgs:
    """Args of a GroupedOps: a View for alpha/beta, a GroupedSpec for grouped roles and
    a list of Views for TensorList roles."""

    def __init__(self, ops: GroupedOps, values: dict, compute_type: int):
        self.lib = ops.lib
        self.values = values  # keep alive until the Plan binds them
        self.handle = _H()
        check(self.lib.ftrainArgsCreate(ctypes.byref(self.handle), ops.ops), "ftrainArgsCreate", self.lib)
        self._lists = []
        for role, v in values.items():
            rid, kind = ops.ids[role], ops.kinds[role]
            if kind == "tensor":
                st = self.lib.ftrainArgsSetTensor(self.handle, rid, v.sv)
            elif kind == "list":
                arr = (StorageView * max(len(v), 1))(*[x.sv for x in v])
                self._lists.append(arr)
                st = self.lib.ftrainArgsSetTensorList(self.handle, rid, arr, len(v))
            else:
                st = self.lib.ftrainArgsSetGroupedTensor(
                    self.handle, rid, v.num_groups, v.data.sv,
                    ctypes.byref(v.offset_view.sv) if v.offset_view is not None else None,
                    v.dim_views, v.stride_views)
            check(st, f"ftrainArgsSet({role})", self.lib)
        set_op = {"abcd": self.lib.ftrainArgsSetGroupedABCDGemm, "bcd": self.lib.ftrainArgsSetGroupedBCDGemm,
                  "ab": self.lib.ftrainArgsSetGroupedABGemm}[ops.kind]
        check(set_op(self.handle, ops.op_id, compute_type), "ftrainArgsSetGrouped*Gemm", self.lib)

    def plan(self) -> Plan:
        h = _H()
        check(self.lib.ftrainPlanCreate(ctypes.byref(h), self.handle), "ftrainPlanCreate", self.lib)
        return Plan(h, self.lib)

    def plan_status_on_device(self, device: int = 0):
        """Plan creation for an explicit device id through the testing library (CPU hosts)."""
        h = _H()
        st = self.lib.ftrainTestingPlanCreateOnDevice(ctypes.byref(h), self.handle, device)
        return st, last_message(self.lib), (Plan(h, self.lib) if st == SUCCESS else None)

    def close(self) -> None:
        if self.handle:
            self.lib.ftrainArgsDestroy(self.handle)
            self.handle = _H()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
