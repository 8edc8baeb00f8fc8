"""RMSNorm forward entry (reference: kernels/triton/rmsnorm.py:46-75).

Backed by the lc_rmsnorm_fwd HIP kernel: one workgroup per row, 16-byte
loads, fp32 sum of squares, any hidden size (the reference's Triton kernel
left columns past 4096 unwritten).
"""
from __future__ import annotations

import torch

from llm_cuda.kernels import _ops


def triton_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return _ops.rms_norm(x, weight, eps)
