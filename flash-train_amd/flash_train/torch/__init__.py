"""flash-train PyTorch binding: ``flash_train.torch.gemm``.

Same signature, checks and defaults as the reference binding
(python/flash_train/torch/csrc/flash_train_torch.cpp:34-75):
``gemm(a, b, c=None, alpha=1.0, beta=0.0) -> d`` with a (m x k), b (k x n)
and optional c (m x n) fp32, rank-2, contiguous device tensors; d is
allocated with ``torch.empty`` and computed on the current stream.
RuntimeError on any violated check.

The native extension is required: importing this module without it raises
(there is no CPU or eager fallback).
"""

import ctypes
import os

import torch  # must load first: it brings the HIP runtime the library shares

_pkg = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ctypes.CDLL(os.path.join(_pkg, "libflash_train.so"), mode=ctypes.RTLD_GLOBAL)

try:
    from ._flash_train_torch import gemm  # noqa: E402
except ModuleNotFoundError as exc:  # pragma: no cover - build problem
    if exc.name != "flash_train.torch._flash_train_torch":
        raise
    raise RuntimeError(
        "flash_train.torch: the native extension is not built; run `python flash-train_amd/build.py`"
    ) from exc

__all__ = ["gemm"]
