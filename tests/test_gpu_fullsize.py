"""GPU parity at the benchmark configurations' full sizes.

The oracle cannot recompute a whole config-3 prefill in seconds, so these tests
compare exactly what it can: every output of configs 2 and 5 (ragged or long
sequences, random page tables), and, at the full config-3 shape (batch 4,
S 4096, 32/8 heads, D 128), sampled rows of the forward and sampled rows/keys
of the backward, each recomputed by the oracle from the inputs it depends on (a
query row needs keys 0..i; a key needs every query row that sees it). Every
row, key and gradient of config 3 is then checked against a plain fp32 PyTorch
recomputation on the device (materialised scores per kv group), itself checked
against the oracle at sampled rows in the same test, to the same bounds.
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


def _fp32_group(q, k, v, b, kvh, G, do=None):
    """Materialised fp32 causal attention of kv group (b, kvh): out [G, S, D],
    lse [G, S]; with do, also dq [G, S, D], dk and dv [S, D] by autograd."""
    D = q.shape[-1]
    qg = q[b, kvh * G:(kvh + 1) * G].float().requires_grad_(do is not None)
    kg = k[b, kvh].float().requires_grad_(do is not None)
    vg = v[b, kvh].float().requires_grad_(do is not None)
    S = qg.shape[1]
    s = torch.matmul(qg, kg.t().contiguous()) * (1.0 / math.sqrt(D))
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool, device=q.device).triu(1), -math.inf)
    lse = torch.logsumexp(s, dim=-1)
    out = torch.matmul(torch.exp(s - lse[..., None]), vg)
    if do is None:
        return out.detach(), lse.detach()
    out.backward(do[b, kvh * G:(kvh + 1) * G].float())
    return out.detach(), lse.detach(), qg.grad, kg.grad, vg.grad


def _max_err(got, ref):
    return (got.float() - ref).abs().max().item()


def test_prefill_config3_all_rows_fp32(cuda):
    """Every row of the config-3 forward against the fp32 recomputation (out
    max-abs 2e-2, lse relative 1e-3); the recomputation itself matches the
    oracle at sampled rows of the first group."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    q, k, v = _config3(cuda)
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    out, lse = triton_fused_causal_attention(q, k, v, return_lse=True)
    qc, kc, vc = q[:1, :G].cpu(), k[:1, :1].cpu(), v[:1, :1].cpu()
    for b in range(B):
        for kvh in range(Hkv):
            ref, ref_lse = _fp32_group(q, k, v, b, kvh, G)
            if b == 0 and kvh == 0:
                for i in (0, 63, 2048, 4095):
                    o_ref, l_ref = causal_attention(qc[:, :, i:i + 1], kc[:, :, :i + 1],
                                                    vc[:, :, :i + 1], q_offset=i)
                    assert _max_err(ref[None, :, i:i + 1].cpu(), o_ref.float()) < 1e-4
                    assert (l_ref.float() - ref_lse[None, :, i:i + 1].cpu()).abs().max() < 1e-4
            got = out[b, kvh * G:(kvh + 1) * G]
            err = _max_err(got, ref)
            assert err <= ATOL[torch.bfloat16], f"out (b {b}, kv head {kvh}): {err:.3e}"
            rel = ((lse[b, kvh * G:(kvh + 1) * G] - ref_lse).abs() / ref_lse.abs().clamp_min(1.0))
            assert rel.max().item() <= 1e-3, f"lse (b {b}, kv head {kvh}): {rel.max().item():.3e}"


def test_backward_config3_all_rows_fp32(cuda):
    """Every dq row and every dk/dv key of config 3 against fp32 autograd of the
    materialised attention (|err| <= 2e-2 * max(1, max |ref|) per tensor and kv
    group); the autograd reference matches the oracle at sampled rows/keys."""
    from llm_cuda.kernels import _ops

    q, k, v = _config3(cuda)
    B, Hq, S, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    g = torch.Generator(device=cuda).manual_seed(1)
    do = torch.randn(q.shape, generator=g, device=cuda, dtype=torch.bfloat16)
    out, lse = _ops.prefill_attention(q, k, v, return_lse=True)
    dq, dk, dv = _ops.prefill_attention_backward(q, k, v, out, lse, do)
    for b in range(B):
        for kvh in range(Hkv):
            _, _, rdq, rdk, rdv = _fp32_group(q, k, v, b, kvh, G, do)
            if b == 0 and kvh == 0:
                qc, kc, vc = q[:1, :G].cpu(), k[:1, :1].cpu(), v[:1, :1].cpu()
                doc = do[:1, :G].cpu()
                i = 2048
                odq, _, _ = causal_attention_backward(qc[:, :, i:i + 1], kc[:, :, :i + 1],
                                                      vc[:, :, :i + 1], doc[:, :, i:i + 1],
                                                      q_offset=i)
                assert _max_err(rdq[None, :, i:i + 1].cpu(), odq.float()) < 1e-3
                j0 = S - 64
                _, odk, odv = causal_attention_backward(qc[:, :, j0:], kc, vc, doc[:, :, j0:],
                                                        q_offset=j0)
                assert _max_err(rdk[None, None, j0:].cpu(), odk[:, :, j0:].float()) < 1e-3
                assert _max_err(rdv[None, None, j0:].cpu(), odv[:, :, j0:].float()) < 1e-3
            for name, got, ref in (("dq", dq[b, kvh * G:(kvh + 1) * G], rdq),
                                   ("dk", dk[b, kvh], rdk), ("dv", dv[b, kvh], rdv)):
                bound = ATOL[torch.bfloat16] * max(1.0, ref.abs().max().item())
                err = _max_err(got, ref)
                assert err <= bound, f"{name} (b {b}, kv head {kvh}): {err:.3e} > {bound:.3e}"
