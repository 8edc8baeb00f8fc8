"""Pins the RMSNorm, SwiGLU and RoPE oracles against independent formulations."""
import math

import torch

from oracle.elementwise import apply_rope, build_inv_freq, build_rope_cache, rms_norm, swiglu


def test_rope_equals_complex_rotation():
    """x*cos + rotate_half(x)*sin == (x1 + i x2) * exp(i theta) per pair (d, d + D/2)."""
    g = torch.Generator().manual_seed(99)
    B, H, S, D = 2, 3, 5, 8
    x = torch.randn(B, H, S, D, generator=g, dtype=torch.float64)
    theta = torch.randn(S, D // 2, generator=g, dtype=torch.float64)
    cos = torch.cat([theta.cos(), theta.cos()], -1)
    sin = torch.cat([theta.sin(), theta.sin()], -1)
    z = torch.complex(x[..., : D // 2], x[..., D // 2:]) * torch.exp(1j * theta)
    expect = torch.cat([z.real, z.imag], -1)
    assert torch.allclose(apply_rope(x, cos, sin).double(), expect, atol=1e-6)


def test_rope_full_width_tables_are_used():
    """With unequal halves (random tables, the reference's GPU tests), the second
    half uses cos/sin[:, D/2:] (x2*c2 + x1*s2)."""
    g = torch.Generator().manual_seed(99)
    x = torch.randn(1, 1, 3, 4, generator=g)
    cos = torch.randn(3, 4, generator=g)
    sin = torch.randn(3, 4, generator=g)
    out = apply_rope(x, cos, sin)
    x1, x2 = x[..., :2], x[..., 2:]
    assert torch.allclose(out[..., :2], x1 * cos[:, :2] - x2 * sin[:, :2])
    assert torch.allclose(out[..., 2:], x2 * cos[:, 2:] + x1 * sin[:, 2:])


def test_rope_tables_position_zero_identity_and_norm():
    cos, sin = build_rope_cache(16, 32, 500000.0, torch.float32)
    assert torch.equal(cos[0], torch.ones(32)) and torch.equal(sin[0], torch.zeros(32))
    assert torch.equal(cos[:, :16], cos[:, 16:]) and torch.equal(sin[:, :16], sin[:, 16:])
    x = torch.randn(1, 2, 16, 32)
    y = apply_rope(x, cos, sin)
    assert torch.allclose(y[:, :, 0], x[:, :, 0])
    n_in = x[..., :16] ** 2 + x[..., 16:] ** 2
    n_out = y[..., :16] ** 2 + y[..., 16:] ** 2
    assert torch.allclose(n_in, n_out, atol=1e-5)


def test_inv_freq_closed_form_and_offset():
    inv = build_inv_freq(8, 10000.0)
    assert torch.allclose(inv, torch.tensor([10000.0 ** (-i / 8) for i in range(0, 8, 2)]))
    cos_a, sin_a = build_rope_cache(4, 8, 10000.0, torch.float32, position_offset=3)
    cos_b, sin_b = build_rope_cache(7, 8, 10000.0, torch.float32)
    assert torch.allclose(cos_a, cos_b[3:]) and torch.allclose(sin_a, sin_b[3:])
    assert abs(float(cos_b[5, 1]) - math.cos(5 * 10000.0 ** (-2 / 8))) < 1e-6


def test_rms_norm_closed_forms():
    c, eps = 3.0, 1e-5
    x = torch.full((2, 7), c)
    w = torch.linspace(0.5, 2.0, 7)
    assert torch.allclose(rms_norm(x, w, eps), c * w / math.sqrt(c * c + eps), atol=1e-6)
    g = torch.Generator().manual_seed(40)
    x = torch.randn(3, 11, generator=g)
    w = torch.randn(11, generator=g)
    for r in range(3):
        ms = sum(float(v) ** 2 for v in x[r]) / 11
        for j in range(11):
            ref = float(x[r, j]) / math.sqrt(ms + eps) * float(w[j])
            assert abs(float(rms_norm(x, w, eps)[r, j]) - ref) < 1e-5


def test_swiglu_closed_forms():
    g = torch.tensor([0.0, 30.0, -30.0, 1.0, -2.5])
    u = torch.tensor([5.0, 2.0, 7.0, 3.0, 1.5])
    out = swiglu(g, u)
    assert out[0] == 0.0
    assert abs(float(out[1]) - 60.0) < 1e-4
    assert abs(float(out[2])) < 1e-10
    for i in (3, 4):
        gv, uv = float(g[i]), float(u[i])
        assert abs(float(out[i]) - gv / (1 + math.exp(-gv)) * uv) < 1e-6
