"""CPU checks of the concatenated projection weights (models/llama3/fused.py)."""
import torch
import torch.nn as nn

from llm_cuda.models.llama3.fused import FusedLinearWeights


def _linears():
    torch.manual_seed(0)
    return nn.Linear(16, 8, bias=False), nn.Linear(16, 4, bias=False), nn.Linear(16, 4, bias=False)


def test_fused_weight_is_the_concatenation_and_aliases_the_parameters():
    a, b, c = _linears()
    ref = torch.cat([a.weight, b.weight, c.weight]).detach().clone()
    f = FusedLinearWeights(a, b, c)
    w = f.weight()
    assert torch.equal(w, ref)
    assert a.weight.data_ptr() == w.data_ptr()
    assert b.weight.data_ptr() == w.data_ptr() + 8 * 16 * 4
    assert f.weight() is w  # cached while the aliasing holds
    x = torch.randn(3, 16)
    y = torch.nn.functional.linear(x, w)
    assert torch.allclose(y, torch.cat([a(x), b(x), c(x)], -1), atol=1e-6)


def test_in_place_parameter_updates_reach_the_fused_weight():
    a, b, c = _linears()
    f = FusedLinearWeights(a, b, c)
    w = f.weight()
    with torch.no_grad():
        b.weight.copy_(torch.full_like(b.weight, 2.0))
    assert f.weight() is w and torch.equal(w[8:12], torch.full((4, 16), 2.0))


def test_replaced_or_converted_parameters_trigger_a_rebuild():
    a, b, c = _linears()
    f = FusedLinearWeights(a, b, c)
    w0 = f.weight()
    c.weight = nn.Parameter(torch.ones(4, 16))
    w1 = f.weight()
    assert w1 is not w0 and torch.equal(w1[12:], torch.ones(4, 16))
    for lin in (a, b, c):
        lin.to(torch.float64)
    w2 = f.weight()
    assert w2.dtype == torch.float64 and a.weight.data_ptr() == w2.data_ptr()


def test_usable_only_without_autograd_recording():
    a, b, c = _linears()
    assert not FusedLinearWeights.usable(a, b, c)
    with torch.no_grad():
        assert FusedLinearWeights.usable(a, b, c)
    for lin in (a, b, c):
        lin.weight.requires_grad_(False)
    assert FusedLinearWeights.usable(a, b, c)


def test_column_layout_is_the_transpose_and_aliases_the_parameters():
    """weight(columns=True): W^T stored contiguously, [K, sum N], each
    parameter a transposed column block of it; in-place updates reach it and
    asking for the other layout rebuilds with the same values."""
    a, b, c = _linears()
    ref = torch.cat([a.weight, b.weight, c.weight]).detach().clone()
    f = FusedLinearWeights(a, b, c)
    wt = f.weight(columns=True)
    assert wt.shape == (16, 16) and wt.is_contiguous() and torch.equal(wt, ref.t())
    assert a.weight.shape == (8, 16) and a.weight.stride() == (1, 16)
    assert b.weight.data_ptr() == wt.data_ptr() + 8 * 4
    assert torch.equal(torch.cat([a.weight, b.weight, c.weight]), ref)
    assert f.weight(columns=True) is wt  # cached while the aliasing holds
    x = torch.randn(3, 16)
    assert torch.allclose(x @ wt, torch.cat([a(x), b(x), c(x)], -1), atol=1e-6)
    with torch.no_grad():
        c.weight.copy_(torch.full_like(c.weight, 3.0))
    assert f.weight(columns=True) is wt and torch.equal(wt[:, 12:], torch.full((16, 4), 3.0))
    w = f.weight()  # back to rows: one rebuild, same values
    assert w.is_contiguous() and w.shape == (16, 16) and torch.equal(w[12:], wt[:, 12:].t())
    assert torch.equal(w[:12], ref[:12]) and a.weight.data_ptr() == w.data_ptr()
    assert f.weight(columns=True) is not wt
