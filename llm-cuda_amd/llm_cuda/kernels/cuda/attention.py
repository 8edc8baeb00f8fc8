"""Causal-attention extension wrapper (reference: kernels/cuda/attention.py:1-37)."""
from __future__ import annotations

import torch

from llm_cuda.kernels import _ops


def cuda_causal_attention_extension(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    attention_mask: torch.Tensor | None = None,
) -> torch.Tensor | None:
    """HIP causal attention; None where the reference returned None (mask, host tensors,
    shape mismatch, unsupported dtype)."""
    if attention_mask is not None:
        return None
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return None
    if q.shape != k.shape or q.shape != v.shape or q.dim() != 4:
        return None
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return None
    return _ops.prefill_attention(q, k, v)
