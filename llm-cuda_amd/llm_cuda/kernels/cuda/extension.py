"""Loader of the native kernel library (reference: kernels/cuda/extension.py:13-49).

The reference JIT-compiled a pybind11 extension on first use and returned None
on any failure. Here the library is prebuilt (llm-cuda_amd/build.py) and
loaded through ctypes; `load_cuda_extension` keeps the reference contract of
returning None when no GPU is present, and otherwise returns the loaded
library or raises.
"""
from __future__ import annotations

import torch

from llm_cuda import _native

_LOAD_ERROR: str | None = None


def load_cuda_extension(verbose: bool = False):
    global _LOAD_ERROR
    if not torch.cuda.is_available():
        _LOAD_ERROR = "CUDA is not available"
        return None
    lib = _native.load()
    _LOAD_ERROR = None
    if verbose:
        print(f"loaded {_native.LIB_PATH} (version {lib.lc_version()})")
    return lib


def get_cuda_extension_load_error() -> str | None:
    return _LOAD_ERROR or _native.load_error()
