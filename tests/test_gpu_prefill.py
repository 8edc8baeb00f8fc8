"""GPU parity: causal prefill attention (O and lse) vs the fp32 oracle.

Cases follow the reference's attention tests (test_triton_attention.py,
seeds 0/11) and add native GQA, q_offset (a cached prefix), lengths that are
not tile multiples, every head_dim the entry accepts, and the benchmark config-3
shape (S 4096, 32/8 heads, D 128, RoPE theta 500000) on a head subset.
"""
import pytest
import torch

from helpers import ATOL, assert_close, assert_lse_close, staircase_qkv
from oracle.attention import causal_attention
from oracle.elementwise import apply_rope, build_rope_cache

pytestmark = pytest.mark.gpu


def _qkv(B, Hq, Hkv, Sq, Skv, D, dtype, device, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(dtype).to(device)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype).to(device)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype).to(device)
    return q, k, v


CASES = [
    # B, Hq, Hkv, S, D, dtype
    (2, 4, 4, 8, 16, torch.float32),      # reference CPU-parity shape
    (1, 2, 2, 16, 32, torch.float16),     # reference GPU shape
    (1, 8, 2, 100, 64, torch.bfloat16),
    (2, 8, 2, 257, 128, torch.bfloat16),
    (1, 4, 1, 130, 128, torch.float16),
    (2, 32, 8, 300, 128, torch.bfloat16),
    (1, 4, 2, 70, 48, torch.bfloat16),    # generic path (D not in {64, 128})
    (1, 2, 1, 33, 256, torch.float32),
    (1, 8, 8, 1, 128, torch.bfloat16),    # single token
    (1, 16, 2, 200, 128, torch.bfloat16),  # 8 q heads per kv head (70B grouping)
    (1, 6, 2, 97, 128, torch.float16),     # 3 q heads per kv head
]


@pytest.mark.parametrize("B,Hq,Hkv,S,D,dtype", CASES)
def test_prefill_matches_oracle(cuda, B, Hq, Hkv, S, D, dtype):
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    q, k, v = _qkv(B, Hq, Hkv, S, S, D, dtype, cuda, seed=S + D)
    out, lse = triton_fused_causal_attention(q, k, v, return_lse=True)
    assert out.shape == q.shape and out.dtype == dtype and lse.dtype == torch.float32
    ref, ref_lse = causal_attention(q.cpu(), k.cpu(), v.cpu())
    assert_close(out, ref, ATOL[dtype], "prefill out")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 64), (torch.bfloat16, 128)])
@pytest.mark.parametrize("Sq,Skv", [(1, 77), (5, 128), (64, 200), (130, 131)])
def test_prefill_with_cached_prefix(cuda, dtype, D, Sq, Skv):
    """q_offset = Skv - Sq: the chunked-prefill masking of models/llama3/attention.py:63-89."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    q, k, v = _qkv(2, 8, 2, Sq, Skv, D, dtype, cuda, seed=Sq)
    out, lse = triton_fused_causal_attention(q, k, v, return_lse=True, q_offset=Skv - Sq)
    ref, ref_lse = causal_attention(q.cpu(), k.cpu(), v.cpu(), q_offset=Skv - Sq)
    assert_close(out, ref, ATOL[dtype], "prefill offset")
    assert_lse_close(lse, ref_lse)


def test_prefill_strided_projection_views(cuda):
    """q/k/v as the transposed [B, S, H, D] projection views the model produces."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    g = torch.Generator().manual_seed(12)
    B, S, Hq, Hkv, D = 2, 96, 8, 2, 128
    q = torch.randn(B, S, Hq * D, generator=g).bfloat16().to(cuda).view(B, S, Hq, D).transpose(1, 2)
    k = torch.randn(B, S, Hkv * D, generator=g).bfloat16().to(cuda).view(B, S, Hkv, D).transpose(1, 2)
    v = torch.randn(B, S, Hkv * D, generator=g).bfloat16().to(cuda).view(B, S, Hkv, D).transpose(1, 2)
    out = triton_fused_causal_attention(q, k, v)
    ref, _ = causal_attention(q.cpu(), k.cpu(), v.cpu())
    assert_close(out, ref, ATOL[torch.bfloat16], "prefill strided")


def test_reference_extension_entry(cuda):
    """cuda_causal_attention_extension keeps the reference's equal-shape contract."""
    from llm_cuda.kernels.cuda.attention import cuda_causal_attention_extension

    q, k, v = _qkv(1, 2, 2, 16, 16, 32, torch.float16, cuda, seed=11)
    out = cuda_causal_attention_extension(q, k, v)
    ref, _ = causal_attention(q.cpu(), k.cpu(), v.cpu())
    assert_close(out, ref, ATOL[torch.float16], "ext entry")
    assert cuda_causal_attention_extension(q, k[:, :1], v[:, :1]) is None


def test_reference_sdpa_helper_runs_the_hip_kernel(cuda):
    """_cuda_sdpa_causal_attention (reference attention.py:61-69) keeps its name
    and contract (causal, scale 1/sqrt(D), no mask) and runs the MFMA kernel."""
    from llm_cuda.kernels.triton.attention import _cuda_sdpa_causal_attention

    q, k, v = _qkv(2, 4, 4, 200, 200, 64, torch.bfloat16, cuda, seed=12)
    out = _cuda_sdpa_causal_attention(q, k, v)
    ref, _ = causal_attention(q.cpu(), k.cpu(), v.cpu())
    assert_close(out, ref, ATOL[torch.bfloat16], "sdpa helper")


def test_baseline_prefill_shape_head_subset(cuda):
    """Benchmark config 3: S 4096, D 128, RoPE theta 500000 by the HIP RoPE kernel,
    GQA 4:1; batch 1 and 2 kv-head groups (8 q heads) keep the oracle in seconds."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention
    from llm_cuda.models.llama3.rotary import apply_rotary

    S, D = 4096, 128
    q, k, v = _qkv(1, 8, 2, S, S, D, torch.bfloat16, cuda, seed=0)
    cos, sin = build_rope_cache(S, D, 500000.0, torch.bfloat16)
    qr, kr = apply_rotary(q, k, cos.to(cuda), sin.to(cuda))
    out, lse = triton_fused_causal_attention(qr, kr, v, return_lse=True)
    qo = apply_rope(q.cpu(), cos, sin).bfloat16()
    ko = apply_rope(k.cpu(), cos, sin).bfloat16()
    # RoPE outputs must agree to the bf16 ulp before attention compares them.
    assert_close(qr, qo, ATOL[torch.bfloat16], "rope q", rtol=2 ** -7)
    ref, ref_lse = causal_attention(qr.cpu(), kr.cpu(), v.cpu())
    assert_close(out, ref, ATOL[torch.bfloat16], "prefill 4096")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 64), (torch.bfloat16, 128)])
def test_prefill_more_queries_than_keys(cuda, dtype, D):
    """Sq > Skv with q_offset 0: rows past the last key see every key."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    q, k, v = _qkv(1, 4, 2, 150, 70, D, dtype, cuda, seed=21)
    out, lse = triton_fused_causal_attention(q, k, v, return_lse=True)
    ref, ref_lse = causal_attention(q.cpu(), k.cpu(), v.cpu())
    assert_close(out, ref, ATOL[dtype], "prefill Sq > Skv")
    assert_lse_close(lse, ref_lse)



@pytest.mark.parametrize("dtype,D,Sq,Skv", [
    (torch.bfloat16, 128, 300, 300),
    (torch.float16, 128, 200, 200),
    (torch.bfloat16, 64, 257, 257),
    (torch.bfloat16, 128, 70, 390),   # cached prefix: q_offset 320
    (torch.float32, 128, 150, 150),   # generic kernel
])
def test_prefill_running_max_rescales(cuda, dtype, D, Sq, Skv):
    """The lazy O / l rescale path (a row max growing by more than 2^8)."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    q, k, v = staircase_qkv(1, 8, 2, Sq, Skv, D, dtype, cuda, seed=Skv)
    out, lse = triton_fused_causal_attention(q, k, v, return_lse=True, q_offset=Skv - Sq)
    ref, ref_lse = causal_attention(q.cpu(), k.cpu(), v.cpu(), q_offset=Skv - Sq)
    # the construction does move the last rows' maxima up one step per 64 keys
    # (scores of the first 64 keys are ~0)
    assert ref_lse.max().item() > 6.0 * ((Skv - 1) // 64) - 1.0
    assert_close(out, ref, ATOL[dtype], "prefill rescales")
    assert_lse_close(lse, ref_lse)


def _abi_prefill(q, k, v, q_offset, counters):
    """lc_prefill_attn_fwd through the C ABI with the given counters (None: every
    workgroup's row group from its block id)."""
    import ctypes
    import math

    from llm_cuda import _native
    from llm_cuda.kernels import _ops

    lib = _native.load()
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, Sq, dtype=torch.float32, device=q.device)
    st = lambda t: (ctypes.c_int64 * 4)(*t.stride())  # noqa: E731
    rc = lib.lc_prefill_attn_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(), B, Hq, Hkv, Sq,
        Skv, D, st(q), st(k), st(v), st(o), q_offset, None, None, 0,
        None if counters is None else counters.data_ptr(), 1.0 / math.sqrt(D),
        _native.lc_dtype(q), _ops._stream(q.device))
    _native.check(rc, "lc_prefill_attn_fwd")
    return o, lse


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Skv,D", [
    (2, 32, 8, 2048, 2048, 128),   # 16 units of 64 row groups
    (4, 32, 8, 1024, 3072, 128),   # cached prefix (q_offset 2048)
    (1, 64, 8, 2048, 2048, 128),   # 8 q heads per kv head: two head groups per kv head
    (2, 16, 8, 4096, 4096, 64),    # two rows of 32 per head group (G = 2)
    (2, 32, 8, 2000, 2000, 128),   # 63 row groups, the last one partial
])
def test_dynamic_tail_matches_static_order(cuda, B, Hq, Hkv, Sq, Skv, D):
    """With counters, the lightest quarter of the MFMA kernel's row groups is
    handed out by a ticket as the workgroups start; which workgroup computes a
    row group changes nothing in it, so out and lse equal the static order
    (NULL counters) bit for bit, call after call, with the ticket back at zero
    after every call; the output matches the oracle at sampled rows."""
    from llm_cuda import _native

    q, k, v = _qkv(B, Hq, Hkv, Sq, Skv, D, torch.bfloat16, cuda, seed=B * Sq + D)
    off = Skv - Sq
    counters = torch.zeros(_native.load().lc_prefill_attn_counter_count(), dtype=torch.int32,
                           device=cuda)
    ref_o, ref_lse = _abi_prefill(q, k, v, off, None)
    for call in range(3):
        o, lse = _abi_prefill(q, k, v, off, counters)
        torch.cuda.synchronize()
        assert torch.equal(o, ref_o), f"call {call}: output differs from the static order"
        assert torch.equal(lse, ref_lse), f"call {call}: lse differs from the static order"
        assert int(counters.abs().sum()) == 0, f"call {call}: ticket not returned to zero"
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    for i in (0, 100, Sq // 2, Sq - 1):
        o_ref, l_ref = causal_attention(qc[:, :, i:i + 1], kc[:, :, :off + i + 1],
                                        vc[:, :, :off + i + 1], q_offset=off + i)
        assert_close(ref_o[:, :, i:i + 1], o_ref, ATOL[torch.bfloat16], f"row {i}")
        assert_lse_close(ref_lse[:, :, i:i + 1], l_ref)
