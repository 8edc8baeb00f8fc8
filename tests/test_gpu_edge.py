"""Zero-size inputs through the public entry points: each returns empty
results of the right shapes and dtypes (no launch reaches the device with a
zero-sized grid), and a batch whose sequences are all empty decodes to zero
outputs with -inf lse (the documented behaviour of an empty sequence)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def test_prefill_zero_batch_and_zero_length(cuda):
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    for shape in [(0, 4, 8, 64), (1, 4, 0, 64)]:
        q = torch.zeros(shape, device=cuda, dtype=BF)
        out, lse = triton_fused_causal_attention(q, q.clone(), q.clone(), return_lse=True)
        assert out.shape == shape and out.dtype == BF
        assert lse.shape == shape[:3] and lse.dtype == torch.float32


def test_paged_decode_zero_batch_and_empty_sequences(cuda):
    from llm_cuda.kernels.triton.decode_attention import paged_decode_attention

    pool = torch.zeros(4, 2, 64, 128, device=cuda, dtype=BF)
    for B in (0, 3):
        q = torch.randn(B, 8, 1, 128, device=cuda).to(BF)
        table = torch.zeros(B, 2, dtype=torch.int32, device=cuda)
        lens = torch.zeros(B, dtype=torch.int32, device=cuda)
        out, lse = paged_decode_attention(q, pool, pool, table, lens, return_lse=True)
        assert out.shape == (B, 8, 1, 128) and out.dtype == BF
        assert lse.shape == (B, 8) and lse.dtype == torch.float32
        assert (out == 0).all() and torch.isinf(lse).all() and (lse < 0).all()


def test_elementwise_and_projections_zero_rows(cuda):
    from llm_cuda.kernels import _ops
    from llm_cuda.kernels.triton.rmsnorm import triton_rms_norm
    from llm_cuda.kernels.triton.rope import triton_apply_rope
    from llm_cuda.kernels.triton.swiglu import triton_swiglu

    x = torch.zeros(0, 256, device=cuda, dtype=BF)
    w = torch.ones(256, device=cuda, dtype=BF)
    assert triton_rms_norm(x, w, 1e-5).shape == (0, 256)
    y, s = _ops.add_rms_norm(x, x.clone(), w, 1e-5)
    assert y.shape == s.shape == (0, 256)
    assert triton_swiglu(x, x.clone()).shape == (0, 256)
    t = torch.zeros(0, 64, device=cuda, dtype=BF)
    assert triton_apply_rope(torch.zeros(1, 4, 0, 64, device=cuda, dtype=BF), t, t).shape == \
        (1, 4, 0, 64)
    weight = torch.randn(512, 256, device=cuda).to(BF)
    assert _ops.decode_linear(x, weight).shape == (0, 512)
    ids = _ops.lm_head_argmax(x, torch.randn(100, 256, device=cuda).to(BF))
    assert ids.shape == (0,) and ids.dtype == torch.int64
