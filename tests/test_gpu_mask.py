"""GPU parity of the additive attention mask (the reference's attention_mask).

The reference adds the mask to the scaled scores before the softmax in its
torch paths (kernels/triton/attention.py:457-477, models/llama3/attention.py:
63-89,138-147) and pins it with a key mask on the CPU
(tests/test_triton_attention.py:78-90). Here every attention kernel takes it:
the prefill MFMA kernel (16-bit and fp32 masks, 4-key vector and strided
element loads), the generic prefill kernel, both backward paths, and the
three paged decode kernels. Each is checked against the oracle with the same
mask; a left-padded batch of unequal prompts is also checked against each
prompt run alone, which the mask must make identical.
"""
import math

import pytest
import torch

from helpers import ATOL, assert_close, assert_lse_close
from oracle.attention import causal_attention, causal_attention_backward
from oracle.decode import paged_decode

pytestmark = pytest.mark.gpu


def _qkv(B, Hq, Hkv, Sq, Skv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Sq, D, generator=g).to(dtype)
    k = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype)
    return q, k, v, g


def _run(q, k, v, mask, dev, **kw):
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    return triton_fused_causal_attention(q.to(dev), k.to(dev), v.to(dev),
                                         attention_mask=mask.to(dev), return_lse=True, **kw)


def test_reference_masked_case(cuda):
    """tests/test_triton_attention.py:78-90 of the reference: seed 1, fp32
    [1, 2, 6, 8], a [1, 1, 1, 6] key mask of -1e4 on the last two keys."""
    torch.manual_seed(1)
    q = torch.randn(1, 2, 6, 8)
    k = torch.randn(1, 2, 6, 8)
    v = torch.randn(1, 2, 6, 8)
    mask = torch.zeros((1, 1, 1, 6))
    mask[..., -2:] = -1e4
    out, lse = _run(q, k, v, mask, cuda)
    ref, ref_lse = causal_attention(q, k, v, bias=mask)
    assert_close(out, ref, 1e-5, "reference mask case")
    assert_lse_close(lse, ref_lse)


def _mask(kind, B, Hq, Sq, Skv, g, dtype):
    if kind == "keypad":        # [B, 1, 1, Skv]: -inf on the trailing keys of sequence 1
        m = torch.zeros(B, 1, 1, Skv)
        m[1 % B, ..., Skv - 37:] = float("-inf")
    elif kind == "finfo":       # [B, 1, 1, Skv]: finfo.min on leading keys (left padding)
        m = torch.zeros(B, 1, 1, Skv)
        m[0, ..., :45] = torch.finfo(torch.float32).min
    elif kind == "rows":        # [1, 1, Sq, Skv]: a dense random bias
        m = 2.0 * torch.randn(1, 1, Sq, Skv, generator=g)
    elif kind == "heads":       # [B, Hq, Sq, Skv]: per head, with -1e4 holes
        m = torch.randn(B, Hq, Sq, Skv, generator=g)
        m[torch.rand(B, Hq, Sq, Skv, generator=g) < 0.1] = -1e4
    elif kind == "strided":     # a transposed view: element-wise loads
        m = torch.randn(B, 1, Skv, Sq, generator=g).transpose(-1, -2)
    else:
        raise ValueError(kind)
    return m.to(dtype)


@pytest.mark.parametrize("kind", ["keypad", "finfo", "rows", "heads", "strided"])
@pytest.mark.parametrize("mdt", [torch.bfloat16, torch.float32])
def test_prefill_mfma_masks(cuda, kind, mdt):
    B, Hq, Hkv, S, D = 2, 8, 2, 200, 128
    q, k, v, g = _qkv(B, Hq, Hkv, S, S, D, torch.bfloat16, seed=3)
    mask = _mask(kind, B, Hq, S, S, g, mdt)
    out, lse = _run(q, k, v, mask, cuda)
    ref, ref_lse = causal_attention(q, k, v, bias=mask)
    assert_close(out, ref, ATOL[torch.bfloat16], f"mask {kind}")
    finite = torch.isfinite(ref_lse) & (ref_lse > -1e29)
    assert_lse_close(lse[finite], ref_lse[finite])


@pytest.mark.parametrize("dtype,D,Sq,Skv,off", [
    (torch.float16, 64, 130, 130, 0),      # f16, head_dim 64
    (torch.bfloat16, 128, 61, 190, 129),   # cached prefix, Skv % 4 != 0 (element loads)
    (torch.float32, 64, 70, 70, 0),        # generic kernel
    (torch.bfloat16, 48, 50, 50, 0),       # generic kernel (head_dim 48)
])
def test_prefill_mask_other_paths(cuda, dtype, D, Sq, Skv, off):
    q, k, v, g = _qkv(2, 4, 2, Sq, Skv, D, dtype, seed=D + Sq)
    mask = 1.5 * torch.randn(2, 1, Sq, Skv, generator=g)
    mask[0, :, :, :9] = float("-inf")
    mask = mask.to(dtype)
    out, lse = _run(q, k, v, mask, cuda, q_offset=off)
    ref, ref_lse = causal_attention(q, k, v, q_offset=off, bias=mask)
    assert_close(out, ref, ATOL[dtype], "mask path")
    assert_lse_close(lse, ref_lse)


def test_left_padded_batch_equals_each_prompt_alone(cuda):
    """Three prompts of 50, 128 and 77 tokens, left-padded to 128 with a
    finfo.min key-padding mask: each prompt's rows equal the prompt run alone,
    and pad rows (every visible key masked) average their keys as the
    reference's softmax of equal scores does."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    lens, S, Hq, Hkv, D = [50, 128, 77], 128, 8, 2, 128
    g = torch.Generator().manual_seed(9)
    q = torch.randn(3, Hq, S, D, generator=g).bfloat16()
    k = torch.randn(3, Hkv, S, D, generator=g).bfloat16()
    v = torch.randn(3, Hkv, S, D, generator=g).bfloat16()
    mask = torch.zeros(3, 1, 1, S, dtype=torch.bfloat16)
    for b, n in enumerate(lens):
        mask[b, ..., :S - n] = torch.finfo(torch.bfloat16).min
    out, lse = _run(q, k, v, mask, cuda)
    ref, _ = causal_attention(q, k, v, bias=mask)
    assert_close(out, ref, ATOL[torch.bfloat16], "padded batch")
    for b, n in enumerate(lens):
        alone, alone_lse = triton_fused_causal_attention(
            q[b:b + 1, :, S - n:].to(cuda), k[b:b + 1, :, S - n:].to(cuda),
            v[b:b + 1, :, S - n:].to(cuda), return_lse=True)
        assert_close(out[b:b + 1, :, S - n:], alone.float(), ATOL[torch.bfloat16], f"prompt {b}")
        assert_lse_close(lse[b:b + 1, :, S - n:], alone_lse)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64),
                                     (torch.float32, 32)])
def test_backward_with_mask(cuda, dtype, D):
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    B, Hq, Hkv, S = 2, 4, 2, 150
    q, k, v, g = _qkv(B, Hq, Hkv, S, S, D, dtype, seed=D)
    mask = torch.randn(B, 1, S, S, generator=g)
    mask[1, :, :, :20] = float("-inf")
    mask = mask.to(dtype)
    do = torch.randn(B, Hq, S, D, generator=g).to(dtype)
    qg, kg, vg = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
    triton_fused_causal_attention(qg, kg, vg, attention_mask=mask.to(cuda)).backward(do.to(cuda))
    refs = causal_attention_backward(q, k, v, do, bias=mask)
    for got, ref, name in zip((qg.grad, kg.grad, vg.grad), refs, "qkv"):
        scale = max(1.0, ref.abs().max().item())
        assert_close(got, ref, ATOL[dtype] * scale, f"d{name} with mask")


def _paged(lens, Hq, Hkv, D, P, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    pages = [max(1, math.ceil(n / P)) for n in lens]
    N = sum(pages) + 1
    perm = torch.randperm(N, generator=g).to(torch.int32)
    bt = torch.full((len(lens), max(pages)), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n]
        o += n
    kp = torch.randn(N, Hkv, P, D, generator=g).to(dtype)
    vp = torch.randn(N, Hkv, P, D, generator=g).to(dtype)
    q = torch.randn(len(lens), Hq, 1, D, generator=g).to(dtype)
    return q, kp, vp, bt, torch.tensor(lens, dtype=torch.int32), g


@pytest.mark.parametrize("dtype,P", [(torch.bfloat16, 64), (torch.bfloat16, 48),
                                     (torch.float16, 64), (torch.float32, 64)])
@pytest.mark.parametrize("per_head", [False, True])
@pytest.mark.parametrize("single_split", [False, True])
def test_paged_decode_masks(cuda, dtype, P, per_head, single_split):
    """Rows kernel (P 64), per-lane-page kernel (P 48), generic kernel (fp32);
    with single_split, one split covers the capacity (the multi-wave
    workgroup kernel at P 64); a [B, 1, 1, L] key mask or a [B, Hq, 1, L]
    per-head mask, with -inf, -1e4 and random entries, shorter than the
    longest sequence (later tokens get no mask)."""
    from llm_cuda.kernels.triton.decode_attention import paged_decode_attention

    lens = [700, 1, 64, 1300]
    Hq, Hkv, D = 16, 4, 128
    q, kp, vp, bt, sl, g = _paged(lens, Hq, Hkv, D, P, dtype, seed=P + int(per_head))
    L = 1100
    mask = torch.randn(len(lens), Hq if per_head else 1, 1, L, generator=g)
    mask[0, ..., 100:200] = float("-inf")
    mask[3, ..., :50] = -1e4
    mask = mask.to(dtype if dtype != torch.float16 else torch.float32)
    split = -(-bt.shape[1] * P // 64) * 64 if single_split else None
    out, lse = paged_decode_attention(q.to(cuda), kp.to(cuda), vp.to(cuda), bt.to(cuda),
                                      sl.to(cuda), return_lse=True, attention_mask=mask.to(cuda),
                                      split_tokens=split)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl, bias=mask[:, :, 0])
    assert_close(out, ref, ATOL[dtype], "decode mask")
    assert_lse_close(lse, ref_lse)


def test_model_masked_forward_and_paged_decode(cuda):
    """A left-padded batch through the model with the reference's mask
    convention (finfo.min on pad keys, [B, 1, q_len, kv_len]): the full forward
    against the oracle model with the same mask, then paged decode steps with
    [B, 1, 1, kv_len] masks against the oracle's full recompute."""
    import oracle.model as omodel
    from llm_cuda.models.llama3.config import Llama3Config
    from llm_cuda.models.llama3.kv_cache import PagedKVCache
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = Llama3Config(vocab_size=512, hidden_size=128, intermediate_size=256,
                       num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2)
    torch.manual_seed(4)
    model = Llama3ForCausalLM(cfg).eval()
    lens, S, steps = [9, 16, 12], 16, 3
    ids = torch.randint(0, cfg.vocab_size, (3, S + steps))
    neg = torch.finfo(torch.float32).min

    def mask_for(kv_len, q_len):
        m = torch.zeros(3, 1, q_len, kv_len)
        for b, n in enumerate(lens):
            m[b, ..., :S - n] = neg
        return m

    full_mask = mask_for(S + steps, S + steps)
    ref = omodel.forward(model.state_dict(), cfg, ids, attention_mask=full_mask)
    gm = model.to(cuda)
    with torch.no_grad():
        got = gm(input_ids=ids.to(cuda), attention_mask=full_mask.to(cuda))["logits"]
    assert (got.cpu() - ref).abs().max().item() < 1e-4
    cache = PagedKVCache.create(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                                S + steps, 4, cuda, torch.float32, batch_size=3)
    with torch.no_grad():
        gm(input_ids=ids[:, :S].to(cuda), attention_mask=mask_for(S, S).to(cuda),
           past_key_values=cache, use_cache=True)
        for t in range(steps):
            kv = S + t + 1
            o = gm(input_ids=ids[:, S + t:S + t + 1].to(cuda),
                   attention_mask=mask_for(kv, 1).to(cuda), past_key_values=cache,
                   use_cache=True)["logits"]
            assert (o[:, 0].cpu() - ref[:, S + t]).abs().max().item() < 1e-4, f"step {t}"
