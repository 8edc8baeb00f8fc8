"""ctypes binding of liblcuda_hip.so, the gfx950 kernels of the attention path.

This module is the only place that touches the C ABI (include/lcuda.h). It
replaces the JIT pybind11 extension loader of the reference
(src/llm_cuda/kernels/cuda/extension.py:13-49): the library is prebuilt
in-tree by llm-cuda_amd/build.py, loaded once, and every failure raises —
there is no silent fallback to another implementation.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the kernels must share)

LIB_PATH = Path(__file__).resolve().parent / "liblcuda_hip.so"

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

_TORCH_TO_LC = {
    torch.float32: DTYPE_F32,
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
}

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes), mirroring include/lcuda.h.
_SIGNATURES = {
    "lc_version": (ctypes.c_int, []),
    "lc_last_error": (ctypes.c_char_p, []),
    "lc_rmsnorm_fwd": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, ctypes.c_int,
         ctypes.c_int, _c_p],
    ),
    "lc_add_rmsnorm_fwd": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         ctypes.c_float, ctypes.c_int, ctypes.c_int, _c_p],
    ),
    "lc_swiglu_fwd": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_p],
    ),
    "lc_rope_fwd": (
        ctypes.c_int,
        [_c_p, _c_p, _c_i64, _c_i64p, _c_i64p, _c_p, _c_p, _c_i64, _c_i64p, _c_i64p, _c_p, _c_p,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_p],
    ),
    "lc_prefill_attn_counter_count": (_c_i64, []),
    "lc_prefill_attn_fwd": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64p,
         _c_i64p, _c_i64p, _c_i64p, _c_i64, _c_p, _c_i64p, ctypes.c_int, _c_p, ctypes.c_float,
         ctypes.c_int, _c_p],
    ),
    "lc_prefill_attn_bwd_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "lc_prefill_attn_bwd": (
        ctypes.c_int,
        [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, _c_i64, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_i64p, _c_i64p,
         _c_i64, _c_p, _c_i64p, ctypes.c_int, ctypes.c_float, _c_p, _c_i64, ctypes.c_int, _c_p],
    ),
    "lc_lm_head_argmax_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "lc_lm_head_argmax_counter_count": (_c_i64, []),
    "lc_lm_head_argmax": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p,
         ctypes.c_int, _c_p],
    ),
    "lc_decode_linear_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int]),
    "lc_decode_linear_counter_count": (_c_i64, [_c_i64, ctypes.c_int]),
    "lc_decode_linear": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int,
         ctypes.c_int, _c_p, _c_i64, _c_p, ctypes.c_int, _c_p],
    ),
    "lc_decode_linear_partial_count": (_c_i64, [_c_i64, _c_i64]),
    "lc_decode_linear_partials": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int,
         _c_p],
    ),
    "lc_add_rmsnorm_partials_fwd": (
        ctypes.c_int,
        [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
         _c_i64, ctypes.c_float, ctypes.c_int, ctypes.c_int, _c_p],
    ),
    "lc_paged_decode_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "lc_paged_decode_counter_count": (_c_i64, []),
    "lc_paged_decode_fwd": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
         _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_p,
         _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float,
         ctypes.c_int, _c_p],
    ),
    "lc_paged_decode_fwd_noalloc": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
         _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, ctypes.c_int, _c_p],
    ),
    "lc_paged_kv_append": (
        ctypes.c_int,
        [_c_p, _c_p, _c_i64p, _c_i64p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64,
         _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_p],
    ),
    "lc_rope_kv_append": (
        ctypes.c_int,
        [_c_p, _c_i64p, _c_p, _c_i64p, _c_p, _c_i64p, _c_p, _c_i64p, _c_p, _c_p, _c_i64, _c_i64,
         _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_p],
    ),
    "lc_paged_decode_step": (
        ctypes.c_int,
        [_c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64,
         _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p,
         _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_float, ctypes.c_int, _c_p],
    ),
    "lc_paged_kv_gather": (
        ctypes.c_int,
        [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64,
         _c_i64, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_p],
    ),
}

EXPORTS = tuple(_SIGNATURES)

_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None
_LOAD_ERROR: str | None = None


class NativeError(RuntimeError):
    """A kernel entry point rejected its arguments or failed to launch."""


def load() -> ctypes.CDLL:
    """Load the library once; raise NativeError if it is missing or broken."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not LIB_PATH.exists():
            _LOAD_ERROR = f"{LIB_PATH} not built (run python llm-cuda_amd/build.py)"
            raise NativeError(_LOAD_ERROR)
        try:
            lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_LOCAL)
            for name, (restype, argtypes) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
        except (OSError, AttributeError) as exc:
            _LOAD_ERROR = f"failed to load {LIB_PATH}: {exc}"
            raise NativeError(_LOAD_ERROR) from exc
        _LIB = lib
        _LOAD_ERROR = None
        return lib


def load_error() -> str | None:
    return _LOAD_ERROR


def status() -> str:
    """'loaded' or 'failed: <reason>' (cf. kernels/cuda/rmsnorm.py:38-46 of the reference)."""
    try:
        load()
    except NativeError as exc:
        return f"failed: {exc}"
    return "loaded"


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().lc_last_error()
        text = msg.decode(errors="replace") if msg else ""
        raise NativeError(f"{what} failed (status {rc}): {text}")


def lc_dtype(t: torch.Tensor) -> int:
    try:
        return _TORCH_TO_LC[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, float16 or bfloat16")


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; returns it.

    The HIP kernels are the only implementation of the attention path: host
    (CPU) tensors are rejected instead of being computed another way.
    """
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "llm_cuda kernels run on ROCm devices only; got a tensor on "
                f"{t.device}. Move inputs to the GPU (there is no CPU implementation)."
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no tensor given")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def strides4(t: torch.Tensor):
    arr = (ctypes.c_int64 * 4)(*t.stride())
    return arr


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
