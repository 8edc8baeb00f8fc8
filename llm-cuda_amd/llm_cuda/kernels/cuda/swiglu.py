"""SwiGLU extension wrapper (reference: kernels/cuda/swiglu.py:1-26)."""
from __future__ import annotations

import torch

from llm_cuda.kernels import _ops


def cuda_swiglu_extension(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor | None:
    """HIP SwiGLU; None for host tensors or non-matching shapes (reference contract)."""
    if not gate.is_cuda or not up.is_cuda:
        return None
    if gate.shape != up.shape:
        return None
    if gate.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return None
    return _ops.swiglu(gate, up)
