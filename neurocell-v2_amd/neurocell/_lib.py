"""Loader for the gfx950 native library and device-tensor plumbing for ctypes calls.

The product path has no CPU or PyTorch fallback: if ``libneurocell_hip.so`` is absent or no
HIP device is visible, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _abi
from ._abi import NeurocellError

LIB_NAME = "libneurocell_hip.so"
_LIB = None


def lib_path() -> str:
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Loads (once) and type-declares the native library; raises if it is missing."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or lib_path()
    if not os.path.exists(p):
        raise NeurocellError(
            f"native library {p} is not built; run __graft_entry__.build() (hipcc, gfx950)")
    lib = _abi.declare(ctypes.CDLL(p))
    if path is None:
        _LIB = lib
    return lib


def lib() -> ctypes.CDLL:
    return load_library()


def require_device() -> torch.device:
    if not torch.cuda.is_available():
        raise NeurocellError("no HIP device visible: the neurocell MI355X path needs a GPU")
    return torch.device("cuda", torch.cuda.current_device())


def stream_ptr() -> ctypes.c_void_p:
    """The current torch (HIP) stream as a raw hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise NeurocellError("expected a device tensor")
    if not t.is_contiguous():
        raise NeurocellError("expected a contiguous tensor")
    return ctypes.c_void_p(t.data_ptr())


def f32(t: torch.Tensor) -> torch.Tensor:
    """Validates an fp32 contiguous device operand (no implicit host copies)."""
    if not t.is_cuda:
        raise NeurocellError("expected a device tensor")
    if t.dtype != torch.float32:
        raise NeurocellError(f"expected float32, got {t.dtype}")
    return t.contiguous()


def call(name: str, *args) -> None:
    L = lib()
    _abi.check(L, getattr(L, name)(*args), name)
