"""RMSNorm, SwiGLU and RoPE oracles (fp32 on the host). TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """models/llama3/norm.py:31-33 and kernels/cuda/rmsnorm.py:6-8, in fp32:
    x * rsqrt(mean(x^2, -1) + eps) * w."""
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    return xf * torch.rsqrt(var + eps) * weight.float()


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """kernels/triton/swiglu.py:103-107 in fp32: (g * sigmoid(g)) * u."""
    g = gate.float()
    return (g * torch.sigmoid(g)) * up.float()


def build_inv_freq(head_dim: int, base: float) -> torch.Tensor:
    """models/llama3/rotary.py:6-26: 1 / base^(arange(0, D, 2) / D), fp32."""
    return 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))


def build_rope_cache(seq_len: int, head_dim: int, base: float, dtype: torch.dtype,
                     position_offset: int = 0, inv_freq: torch.Tensor | None = None):
    """models/llama3/rotary.py:29-71: positions (fp32) outer inv_freq, cat(f, f),
    cos/sin cast to dtype. An inv_freq of another dtype (a bf16 model's buffer)
    is used as given, as torch.outer does in the reference."""
    if inv_freq is None:
        inv_freq = build_inv_freq(head_dim, base)
    pos = torch.arange(position_offset, position_offset + seq_len, dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq.cpu())
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """models/llama3/rotary.py:74-78: cat(-x2, x1)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """models/llama3/rotary.py:104-109 (fallback) in fp32 with full-width tables:
    x * cos + rotate_half(x) * sin; x [B, H, S, D], cos/sin [S, D]."""
    xf = x.float()
    return xf * cos.float() + rotate_half(xf) * sin.float()
