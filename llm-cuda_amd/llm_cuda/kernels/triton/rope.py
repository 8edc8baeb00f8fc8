"""Fused RoPE forward entry (reference: kernels/triton/rope.py:128-222).

`triton_apply_rope(x, cos, sin)` returns x*cos + rotate_half(x)*sin for
x [B, H, S, D] (any strides, e.g. the transposed projection views: no
.contiguous() copy is made) and FULL-width [S, D] tables. `apply_rope_qk`
rotates Q and K in one launch.
"""
from __future__ import annotations

import torch

from llm_cuda.kernels import _ops

_MAX_HEAD_DIM = 256


def can_use_triton_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> bool:
    """Same guards as the reference (rope.py:128-153): device tensors, f16/bf16/f32,
    4-D x, even head_dim, [S, D] tables."""
    if not (x.is_cuda and cos.is_cuda and sin.is_cuda):
        return False
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    if x.dim() != 4 or cos.dim() != 2 or sin.dim() != 2:
        return False
    head_dim = x.shape[-1]
    if head_dim % 2 != 0 or head_dim > _MAX_HEAD_DIM:
        return False
    if cos.shape != sin.shape:
        return False
    if cos.shape != (x.shape[-2], head_dim):
        return False
    if cos.dtype != x.dtype or sin.dtype != x.dtype:
        return False
    return True


def triton_apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    out, _ = _ops.rope(x, cos, sin)
    return out


def apply_rope_qk(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """Rotate q [B, Hq, S, D] and k [B, Hkv, S, D] in a single kernel launch."""
    return _ops.rope(q, cos, sin, k)
