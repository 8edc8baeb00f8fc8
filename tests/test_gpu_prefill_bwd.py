"""GPU parity: causal attention backward (dq, dk, dv) vs the fp32 oracle.

The oracle (oracle.attention.causal_attention_backward) is pinned against
fp64 autograd and finite differences in test_oracle_attention.py. Cases follow
the reference's backward tests (test_triton_attention.py:94-163: fp32
(2, 3, 8, 16) and f16 (1, 2, 16, 32), seed 11) and add native GQA, q_offset,
lengths that are not tile multiples, the generic head dims, and a benchmark-like
head subset.

Tolerance: gradients scale with their own magnitude (a bf16 operand carries a
2^-9 relative rounding), so the bound is |out - ref| <= atol * max(1, max|ref|)
with atol the forward's per-dtype bound (bf16 2e-2, f16 1e-2, fp32 1e-4).
"""
import pytest
import torch

from helpers import ATOL, staircase_qkv
from oracle.attention import causal_attention_backward

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, Sq, Skv, D, dtype, device, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(dtype).to(device)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype).to(device)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype).to(device)
    do = torch.randn(B, Hq, Sq, D, generator=g).to(dtype).to(device)
    return q, k, v, do


def _assert_grad_close(out, ref, dtype, what):
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert o.shape == r.shape, f"{what}: shape {tuple(o.shape)} != {tuple(r.shape)}"
    assert torch.isfinite(o).all(), f"{what}: non-finite values"
    if not r.numel():
        return
    bound = ATOL[dtype] * max(1.0, r.abs().max().item())
    err = (o - r).abs().max().item()
    assert err <= bound, f"{what}: max abs err {err:.3e} > {bound:.3e}"


def _check(q, k, v, do, q_offset, dtype):
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = triton_fused_causal_attention(qg, kg, vg, q_offset=q_offset)
    out.backward(do)
    rdq, rdk, rdv = causal_attention_backward(q.cpu(), k.cpu(), v.cpu(), do.cpu(),
                                              q_offset=q_offset)
    for name, got, ref in (("dq", qg.grad, rdq), ("dk", kg.grad, rdk), ("dv", vg.grad, rdv)):
        assert got.dtype == dtype
        _assert_grad_close(got, ref, dtype, name)


CASES = [
    # B, Hq, Hkv, S, D, dtype
    (2, 3, 3, 8, 16, torch.float32),      # reference CPU backward shape
    (1, 2, 2, 16, 32, torch.float16),     # reference GPU backward shape
    (1, 4, 4, 64, 64, torch.bfloat16),
    (1, 8, 2, 100, 64, torch.bfloat16),
    (2, 8, 2, 257, 128, torch.bfloat16),
    (1, 4, 1, 130, 128, torch.float16),
    (1, 4, 2, 70, 48, torch.bfloat16),
    (1, 2, 1, 33, 256, torch.float32),
    (1, 8, 8, 1, 128, torch.bfloat16),
    (1, 6, 2, 200, 128, torch.float16),   # G = 3: one head per wave group
    (2, 16, 2, 129, 64, torch.bfloat16),  # G = 8
    (1, 2, 2, 64, 96, torch.bfloat16),    # D padded to 128 on the MFMA path
]


@pytest.mark.parametrize("B,Hq,Hkv,S,D,dtype", CASES)
def test_backward_matches_oracle(cuda, B, Hq, Hkv, S, D, dtype):
    q, k, v, do = _inputs(B, Hq, Hkv, S, S, D, dtype, cuda, seed=S + D + 11)
    _check(q, k, v, do, 0, dtype)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 64), (torch.bfloat16, 128)])
@pytest.mark.parametrize("Sq,Skv", [(1, 77), (5, 128), (64, 200), (130, 131)])
def test_backward_with_cached_prefix(cuda, dtype, D, Sq, Skv):
    q, k, v, do = _inputs(2, 8, 2, Sq, Skv, D, dtype, cuda, seed=Sq + 3)
    _check(q, k, v, do, Skv - Sq, dtype)


def test_backward_reference_gpu_case_seed11(cuda):
    """The reference's f16 case with its tolerances (atol 3e-2, rtol 6e-2)."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    torch.manual_seed(11)
    shape = (1, 2, 16, 32)
    q, k, v, do = (torch.randn(*shape).half().to(cuda) for _ in range(4))
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    (triton_fused_causal_attention(qg, kg, vg) * do).sum().backward()
    rdq, rdk, rdv = causal_attention_backward(q.cpu(), k.cpu(), v.cpu(), do.cpu())
    for got, ref in ((qg.grad, rdq), (kg.grad, rdk), (vg.grad, rdv)):
        assert torch.allclose(got.float().cpu(), ref, atol=3e-2, rtol=6e-2)


def test_backward_strided_inputs_and_ops_entry(cuda):
    """Transposed projection views through the _ops entry; grads are [B, H, S, D]."""
    from llm_cuda.kernels import _ops

    g = torch.Generator().manual_seed(5)
    B, S, Hq, Hkv, D = 2, 96, 8, 2, 128
    mk = lambda h: torch.randn(B, S, h * D, generator=g).bfloat16().to(cuda).view(B, S, h, D).transpose(1, 2)  # noqa: E731
    q, k, v, do = mk(Hq), mk(Hkv), mk(Hkv), mk(Hq)
    out, lse = _ops.prefill_attention(q, k, v, return_lse=True)
    dq, dk, dv = _ops.prefill_attention_backward(q, k, v, out, lse, do)
    rdq, rdk, rdv = causal_attention_backward(q.cpu(), k.cpu(), v.cpu(), do.cpu())
    _assert_grad_close(dq, rdq, torch.bfloat16, "dq")
    _assert_grad_close(dk, rdk, torch.bfloat16, "dk")
    _assert_grad_close(dv, rdv, torch.bfloat16, "dv")


def test_backward_baseline_shape_head_subset(cuda):
    """S 2048, GQA 8:2, D 128 (a slice of the 8B prefill layer's 32:8 heads)."""
    q, k, v, do = _inputs(1, 8, 2, 2048, 2048, 128, torch.bfloat16, cuda, seed=7)
    _check(q, k, v, do, 0, torch.bfloat16)


def test_backward_rejects_bad_lse(cuda):
    from llm_cuda.kernels import _ops

    q, k, v, do = _inputs(1, 2, 2, 8, 8, 64, torch.bfloat16, cuda, seed=1)
    out, lse = _ops.prefill_attention(q, k, v, return_lse=True)
    with pytest.raises(ValueError):
        _ops.prefill_attention_backward(q, k, v, out, lse.half(), do)
    with pytest.raises(ValueError):
        _ops.prefill_attention_backward(q, k, v, out, lse[:, :1], do)


def test_no_grad_path_does_not_record_graph(cuda):
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    q, k, v, _ = _inputs(1, 2, 2, 8, 8, 64, torch.bfloat16, cuda, seed=2)
    out = triton_fused_causal_attention(q, k, v)
    assert out.grad_fn is None


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 64), (torch.bfloat16, 128)])
def test_backward_more_queries_than_keys(cuda, dtype, D):
    """Sq > Skv with q_offset 0: rows past the last key see every key."""
    q, k, v, do = _inputs(1, 4, 2, 150, 70, D, dtype, cuda, seed=21)
    _check(q, k, v, do, 0, dtype)


def test_backward_with_broadcast_output_gradient(cuda):
    """dO from out.sum(): an expanded, stride-0 gradient."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    q, k, v, _ = _inputs(1, 4, 2, 96, 96, 128, torch.bfloat16, cuda, seed=22)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    triton_fused_causal_attention(qg, kg, vg).sum().backward()
    ones = torch.ones(q.shape, dtype=torch.bfloat16)
    rdq, rdk, rdv = causal_attention_backward(q.cpu(), k.cpu(), v.cpu(), ones)
    _assert_grad_close(qg.grad, rdq, torch.bfloat16, "dq")
    _assert_grad_close(kg.grad, rdk, torch.bfloat16, "dk")
    _assert_grad_close(vg.grad, rdv, torch.bfloat16, "dv")


def test_backward_empty_query_or_key_sets(cuda):
    from llm_cuda.kernels import _ops

    q, k, v, do = _inputs(1, 2, 2, 0, 16, 64, torch.bfloat16, cuda, seed=23)
    out, lse = _ops.prefill_attention(q, k, v, return_lse=True)
    dq, dk, dv = _ops.prefill_attention_backward(q, k, v, out, lse, do)
    assert dq.shape == q.shape and dk.shape == k.shape
    # no query row sees any key: dk and dv are zero
    assert dk.abs().max().item() == 0 and dv.abs().max().item() == 0


@pytest.mark.parametrize("dtype,Sq,Skv", [(torch.bfloat16, 300, 300), (torch.bfloat16, 70, 390),
                                          (torch.float32, 150, 150)])
def test_backward_wide_score_range(cuda, dtype, Sq, Skv):
    """Scores that climb by ~8.7 log2 units every 64 keys (the forward's
    rescale-path inputs): P spans many orders of magnitude within a row."""
    q, k, v = staircase_qkv(1, 8, 2, Sq, Skv, 128, dtype, cuda, seed=Skv + 5)
    g = torch.Generator().manual_seed(Skv)
    do = torch.randn(q.shape, generator=g).to(dtype).to(cuda)
    _check(q, k, v, do, Skv - Sq, dtype)
