"""Empty tensors through the reference-named entry points: empty in, empty (or
zero) out, as the torch paths of the reference behave."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_empty_inputs(cuda):
    from llm_cuda.kernels import _ops
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention
    from llm_cuda.kernels.triton.rmsnorm import triton_rms_norm
    from llm_cuda.kernels.triton.rope import triton_apply_rope
    from llm_cuda.kernels.triton.swiglu import triton_swiglu

    bf = torch.bfloat16
    x = torch.empty(0, 4096, device=cuda, dtype=bf)
    w = torch.ones(4096, device=cuda, dtype=bf)
    assert triton_rms_norm(x, w, 1e-5).shape == (0, 4096)
    y, s = _ops.add_rms_norm(x, x.clone(), w, 1e-5)
    assert y.shape == (0, 4096) and s.shape == (0, 4096)
    g = torch.empty(3, 0, device=cuda, dtype=bf)
    assert triton_swiglu(g, g.clone()).shape == (3, 0)
    q = torch.empty(2, 4, 0, 64, device=cuda, dtype=bf)
    cs = torch.empty(0, 64, device=cuda, dtype=bf)
    assert triton_apply_rope(q, cs, cs).shape == q.shape
    out = triton_fused_causal_attention(q, q[:, :2].clone(), q[:, :2].clone())
    assert out.shape == q.shape
    ids = _ops.lm_head_argmax(torch.empty(0, 128, device=cuda, dtype=bf),
                              torch.randn(10, 128, device=cuda, dtype=bf))
    assert ids.shape == (0,) and ids.dtype == torch.int64
