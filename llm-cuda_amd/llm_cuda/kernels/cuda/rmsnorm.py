"""RMSNorm extension wrapper (reference: kernels/cuda/rmsnorm.py:1-46)."""
from __future__ import annotations

import torch

from llm_cuda import _native
from llm_cuda.kernels import _ops

from .extension import get_cuda_extension_load_error, load_cuda_extension


def cuda_rms_norm_extension(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor | None:
    """HIP RMSNorm; None for host tensors (the reference's "not applicable")."""
    if not x.is_cuda or not weight.is_cuda:
        return None
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return None
    return _ops.rms_norm(x, weight, eps)


def cuda_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """HIP RMSNorm; raises for host tensors (no CPU implementation ships)."""
    return _ops.rms_norm(x, weight, eps)


def cuda_extension_status() -> str:
    if load_cuda_extension(verbose=False) is not None:
        return "loaded"
    error = get_cuda_extension_load_error()
    if error is None:
        return _native.status()
    return f"failed: {error}"
