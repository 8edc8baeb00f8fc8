"""Autograd behaviour of the HIP entry points.

The causal attention forward is differentiable (its backward is
lc_prefill_attn_bwd; see test_gpu_prefill_bwd.py). The other kernels of this
inference path (RMSNorm, add + RMSNorm, SwiGLU, RoPE, paged decode, the decode
RoPE + KV append) have no backward here: with autograd recording, their
outputs carry a graph node whose backward raises NotImplementedError, so a
loss.backward() through them fails loudly instead of leaving the parameters
upstream of them without gradients. The reference's SwiGLU is differentiable
(kernels/triton/swiglu.py:91-196); training is outside this build.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _backward_raises(out):
    assert out.requires_grad and out.grad_fn is not None
    with pytest.raises(NotImplementedError, match="no backward"):
        out.float().sum().backward()


def test_elementwise_kernels_raise_on_backward(cuda):
    from llm_cuda.kernels import _ops

    x = torch.randn(4, 64, device=cuda, requires_grad=True)
    w = torch.ones(64, device=cuda, requires_grad=True)
    _backward_raises(_ops.rms_norm(x, w, 1e-5))
    y, s = _ops.add_rms_norm(x, torch.randn(4, 64, device=cuda), w, 1e-5)
    _backward_raises(y)
    _backward_raises(s)
    with pytest.raises(NotImplementedError):
        _ops.add_rms_norm(x, x.detach(), w, 1e-5, inplace=True)
    g = torch.randn(4, 64, device=cuda, requires_grad=True)
    _backward_raises(_ops.swiglu(g, torch.randn(4, 64, device=cuda)))
    q = torch.randn(1, 4, 8, 32, device=cuda, requires_grad=True)
    k = torch.randn(1, 2, 8, 32, device=cuda)
    cos, sin = torch.randn(8, 32, device=cuda), torch.randn(8, 32, device=cuda)
    qo, ko = _ops.rope(q, cos, sin, k)
    _backward_raises(qo)
    assert not ko.requires_grad or ko.grad_fn is not None
    qo1, none = _ops.rope(q, cos, sin)
    assert none is None
    _backward_raises(qo1)


def test_paged_decode_raises_on_backward(cuda):
    from llm_cuda.kernels.triton.decode_attention import triton_decode_attention

    q = torch.randn(2, 4, 1, 64, device=cuda, requires_grad=True)
    k = torch.randn(2, 2, 40, 64, device=cuda)
    v = torch.randn(2, 2, 40, 64, device=cuda)
    _backward_raises(triton_decode_attention(q, k, v))
    out, lse = triton_decode_attention(q, k, v, return_lse=True)
    _backward_raises(out)


def test_no_graph_without_grad(cuda):
    from llm_cuda.kernels import _ops

    x = torch.randn(4, 64, device=cuda, requires_grad=True)
    w = torch.ones(64, device=cuda)
    with torch.no_grad():
        y = _ops.rms_norm(x, w, 1e-5)
    assert not y.requires_grad
    y = _ops.rms_norm(x.detach(), w, 1e-5)
    assert y.grad_fn is None


def test_model_loss_backward_raises(cuda):
    """Llama3ForCausalLM.forward(labels=...) still returns the loss; its backward
    raises rather than silently skipping the parameters upstream of a norm."""
    from llm_cuda.models.llama3.config import Llama3Config
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = Llama3Config(vocab_size=256, hidden_size=64, intermediate_size=128,
                       num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2)
    torch.manual_seed(0)
    model = Llama3ForCausalLM(cfg).to(cuda)
    ids = torch.randint(0, 256, (2, 10), device=cuda)
    out = model(input_ids=ids, labels=ids)
    assert torch.isfinite(out["loss"])
    with pytest.raises(NotImplementedError, match="no backward"):
        out["loss"].backward()
    # inference under no_grad is unaffected
    with torch.no_grad():
        assert model(input_ids=ids)["logits"].grad_fn is None
