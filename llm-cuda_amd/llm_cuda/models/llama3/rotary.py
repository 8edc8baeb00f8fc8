"""RoPE tables and application (reference: models/llama3/rotary.py:1-109).

The tables are built exactly as the reference builds them (fp32 positions,
outer product with `inv_freq`, cat(freqs, freqs), cast to the activation
dtype) so a bf16 model sees the same bf16 tables; when the model is cast to
bf16 its `inv_freq` buffer is bf16 too, and that is what `build_rope_cache`
multiplies by. The rotation itself runs on the HIP RoPE kernel, Q and K in
one launch.
"""
from __future__ import annotations

import torch

from llm_cuda.kernels.triton.rope import apply_rope_qk


def build_inv_freq(head_dim: int, base: float, device: torch.device) -> torch.Tensor:
    """inv_freq[i] = base ** (-2i / head_dim), fp32 [head_dim // 2]."""
    exponents = torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim
    return 1.0 / (base ** exponents)


def build_rope_cache(
    seq_len: int,
    head_dim: int,
    base: float,
    device: torch.device,
    dtype: torch.dtype,
    position_offset: int = 0,
    inv_freq: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """cos, sin [seq_len, head_dim] for positions position_offset .. +seq_len-1."""
    if inv_freq is None:
        inv_freq = build_inv_freq(head_dim, base, device)
    elif inv_freq.device != device:
        inv_freq = inv_freq.to(device=device)
    positions = torch.arange(
        position_offset, position_offset + seq_len, device=device, dtype=torch.float32)
    freqs = torch.outer(positions, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype=dtype), emb.sin().to(dtype=dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary(
    q: torch.Tensor,
    k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor]:
    """q*cos + rotate_half(q)*sin and the same for k, one HIP launch.

    q: [B, Hq, S, D], k: [B, Hkv, S, D] (any strides), cos/sin: [S, D].
    Returns contiguous tensors of the same shapes and dtype.
    """
    return apply_rope_qk(q, k, cos, sin)
