"""Lazy loader of the HIP library ``libr2splat_hip.so``.

Mirrors the reference's lazy extension proxy (r2splat/cuda/_backend.py:10-58):
importing this module never initialises the GPU; the first attribute access
on ``_C`` loads the library (only when a GPU is visible) and fails loudly
with ``RuntimeError`` when it is missing.  There is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import importlib
import os
from typing import Optional

import torch

from ._lib import LIB_PATH, load

__all__ = ["_C", "is_cuda_available", "library"]


class _LazyModule:
    def __init__(self) -> None:
        self._module = None
        self._lib: Optional[ctypes.CDLL] = None
        self._load_attempted = False
        self._error: Optional[str] = None

    def _try_load(self) -> None:
        if self._load_attempted:
            return
        self._load_attempted = True
        if not torch.cuda.is_available():
            self._error = "no GPU is visible (torch.cuda.is_available() is False)"
            return
        if not os.path.exists(LIB_PATH):
            self._error = f"{LIB_PATH} is missing; build it with `python bt-3dgs_amd/build.py`"
            return
        try:
            self._lib = load(LIB_PATH)
            self._module = importlib.import_module("r2splat.cuda._ops")
        except (OSError, AttributeError, RuntimeError) as exc:
            self._error = f"failed to load {LIB_PATH}: {exc}"
            self._lib = None
            self._module = None

    def __getattr__(self, name: str):
        self._try_load()
        if self._module is None:
            raise RuntimeError(f"r2splat HIP library is unavailable: {self._error}")
        return getattr(self._module, name)

    def is_available(self) -> bool:
        self._try_load()
        return self._module is not None

    def library(self) -> ctypes.CDLL:
        self._try_load()
        if self._lib is None:
            raise RuntimeError(f"r2splat HIP library is unavailable: {self._error}")
        return self._lib


_lazy_C = _LazyModule()


class _CProxy:
    def __getattr__(self, name: str):
        return getattr(_lazy_C, name)

    def __bool__(self) -> bool:
        return _lazy_C.is_available()


_C = _CProxy()


def is_cuda_available() -> bool:
    return _lazy_C.is_available()


def library() -> ctypes.CDLL:
    """The loaded ctypes library (raises RuntimeError if unavailable)."""
    return _lazy_C.library()
