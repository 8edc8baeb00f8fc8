"""GPU parity at the benchmark configurations' full sizes.

The oracle cannot recompute a whole config-3 prefill in seconds, so these tests
compare exactly what it can: every output of config 2 (64 ragged sequences,
random page table), and, at the full config-3 shape (batch 4, S 4096, 32/8
heads, D 128), sampled rows of the forward and sampled rows/keys of the
backward, each recomputed by the oracle from the inputs it depends on (a query
row needs keys 0..i; a key needs every query row that sees it).
"""
import math

import pytest
import torch

from helpers import ATOL, assert_close, assert_lse_close
from oracle.attention import causal_attention, causal_attention_backward
from oracle.decode import paged_decode

pytestmark = pytest.mark.gpu


def _config2(device):
    """Benchmark config 2 as bench.py builds it (seed 0)."""
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 8193, (64,), generator=g).tolist()
    P, Hq, Hkv, D = 64, 32, 8, 128
    npages = [math.ceil(n / P) for n in lens]
    N = sum(npages)
    perm = torch.randperm(N, generator=g).to(torch.int32)
    bt = torch.full((64, max(npages)), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(npages):
        bt[b, :n] = perm[o:o + n]
        o += n
    kp = torch.randn(N, Hkv, P, D, generator=g).bfloat16()
    vp = torch.randn(N, Hkv, P, D, generator=g).bfloat16()
    q = torch.randn(64, Hq, 1, D, generator=g).bfloat16()
    return q, kp, vp, bt, torch.tensor(lens, dtype=torch.int32)


def test_decode_config2_all_sequences(cuda):
    from llm_cuda.kernels.triton.decode_attention import paged_decode_attention

    q, kp, vp, bt, sl = _config2(cuda)
    out, lse = paged_decode_attention(q.to(cuda), kp.to(cuda), vp.to(cuda), bt.to(cuda),
                                      sl.to(cuda), return_lse=True)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert_close(out.view(ref.shape), ref, ATOL[torch.bfloat16], "decode config 2")
    assert_lse_close(lse, ref_lse)


def test_decode_config5_all_sequences(cuda):
    """Config 5 exactly as bench.py times it: 8 sequences of 32768 tokens at the
    70B attention shape (64/8 heads, D 128, P 64), block table
    randperm(4096).view(8, 512), the library's default split (4 workgroup
    splits of 8192 tokens per (sequence, kv head)), every output against the
    oracle."""
    from llm_cuda.kernels import _ops
    from llm_cuda.kernels.triton.decode_attention import paged_decode_attention

    B, Hq, Hkv, D, P, L = 8, 64, 8, 128, 64, 32768
    npg = L // P
    g = torch.Generator().manual_seed(0)
    bt = torch.randperm(B * npg, generator=g).to(torch.int32).view(B, npg)
    gd = torch.Generator(device=cuda).manual_seed(0)
    kp = torch.randn(B * npg, Hkv, P, D, generator=gd, device=cuda, dtype=torch.bfloat16)
    vp = torch.randn(B * npg, Hkv, P, D, generator=gd, device=cuda, dtype=torch.bfloat16)
    q = torch.randn(B, Hq, 1, D, generator=gd, device=cuda, dtype=torch.bfloat16)
    sl = torch.full((B,), L, dtype=torch.int32)
    # the split bench.py's config-5 call takes (nothing passed but the tensors)
    split = _ops.choose_split_tokens(B, Hkv, Hq // Hkv, npg * P, P, D, None,
                                     _ops._cu_count(cuda))
    assert split == 8192
    out, lse = paged_decode_attention(q, kp, vp, bt.to(cuda), sl.to(cuda), return_lse=True)
    ref, ref_lse = paged_decode(q.cpu(), kp.cpu(), vp.cpu(), bt, sl)
    assert_close(out.view(ref.shape), ref, ATOL[torch.bfloat16], "decode config 5")
    assert_lse_close(lse, ref_lse)


def _config3(device):
    from llm_cuda.models.llama3.rotary import apply_rotary, build_rope_cache

    B, Hq, Hkv, S, D = 4, 32, 8, 4096, 128
    g = torch.Generator(device=device).manual_seed(0)
    q = torch.randn(B, Hq, S, D, generator=g, device=device, dtype=torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g, device=device, dtype=torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g, device=device, dtype=torch.bfloat16)
    cos, sin = build_rope_cache(S, D, 500000.0, device, torch.bfloat16)
    q, k = apply_rotary(q, k, cos, sin)
    return q, k, v


SAMPLE_ROWS = [0, 1, 31, 32, 63, 64, 1000, 2047, 2048, 3001, 4094, 4095]


def test_prefill_config3_sampled_rows(cuda):
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    q, k, v = _config3(cuda)
    out, lse = triton_fused_causal_attention(q, k, v, return_lse=True)
    out, lse = out.cpu(), lse.cpu()
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    for i in SAMPLE_ROWS:
        ref, ref_lse = causal_attention(qc[:, :, i:i + 1], kc[:, :, :i + 1], vc[:, :, :i + 1],
                                        q_offset=i)
        assert_close(out[:, :, i:i + 1], ref, ATOL[torch.bfloat16], f"prefill row {i}")
        assert_lse_close(lse[:, :, i:i + 1], ref_lse, f"lse row {i}")


def _grad_close(got, ref, what):
    bound = ATOL[torch.bfloat16] * max(1.0, ref.abs().max().item())
    err = (got.float() - ref).abs().max().item()
    assert err <= bound, f"{what}: max abs err {err:.3e} > {bound:.3e}"


def test_backward_config3_sampled(cuda):
    """dq at sampled query rows; dk/dv at every key of the last 128 positions
    (their gradients need only the query rows from that point on)."""
    from llm_cuda.kernels import _ops

    q, k, v = _config3(cuda)
    g = torch.Generator(device=cuda).manual_seed(1)
    do = torch.randn(q.shape, generator=g, device=cuda, dtype=torch.bfloat16)
    out, lse = _ops.prefill_attention(q, k, v, return_lse=True)
    dq, dk, dv = _ops.prefill_attention_backward(q, k, v, out, lse, do)
    dq, dk, dv = dq.cpu(), dk.cpu(), dv.cpu()
    qc, kc, vc, doc = q.cpu(), k.cpu(), v.cpu(), do.cpu()
    S = q.shape[2]
    for i in (0, 1, 63, 64, 2048, 4095):
        rdq, _, _ = causal_attention_backward(qc[:, :, i:i + 1], kc[:, :, :i + 1],
                                              vc[:, :, :i + 1], doc[:, :, i:i + 1], q_offset=i)
        _grad_close(dq[:, :, i:i + 1], rdq, f"dq row {i}")
    j0 = S - 128
    _, rdk, rdv = causal_attention_backward(qc[:, :, j0:], kc, vc, doc[:, :, j0:], q_offset=j0)
    _grad_close(dk[:, :, j0:], rdk[:, :, j0:], "dk last 128 keys")
    _grad_close(dv[:, :, j0:], rdv[:, :, j0:], "dv last 128 keys")
