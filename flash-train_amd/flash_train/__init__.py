"""flash-train for MI355X: the FP32 GEMM family path behind the flash-train API.

`flash_train.torch` holds the PyTorch binding (reference
python/flash_train/__init__.py:10-18 exposes it the same lazy way);
`flash_train.capi` is a ctypes mirror of the C ABI in include/flash_train.
"""

import importlib
import typing


def __getattr__(name: str) -> typing.Any:
    if name in ("torch", "capi"):
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


__all__ = ["torch", "capi"]
