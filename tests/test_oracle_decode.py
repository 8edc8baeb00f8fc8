"""Pins oracle.decode (decode attention, page gather, split merge).

decode_attention: equals the last row of the independently pinned prefill
oracle; kv_len = 1 gives v (tests/test_triton_decode_attention.py:247-258);
fp64 per-(b, h) loop at seed 42 (the reference's _reference_decode_attention
shapes, :177-184). gather_pages: identity table == the reference's get_kv
concat-of-pages semantics (kv_cache.py:65-83, restated as a loop over pages);
random permutation == element-by-element brute force. merge_splits: the
merged result does not depend on how the keys are split.
"""
import math

import numpy as np
import pytest
import torch

from oracle.attention import causal_attention
from oracle.decode import decode_attention, gather_pages, gather_pages_torch, merge_splits, paged_decode


@pytest.mark.parametrize("B,Hq,Hkv,L,D", [(2, 4, 4, 16, 16), (1, 8, 4, 32, 16), (3, 6, 2, 9, 8)])
def test_decode_equals_last_prefill_row(B, Hq, Hkv, L, D):
    torch.manual_seed(42)
    q = torch.randn(B, Hq, L, D)
    k = torch.randn(B, Hkv, L, D)
    v = torch.randn(B, Hkv, L, D)
    o_full, l_full = causal_attention(q, k, v)
    o, lse = decode_attention(q[:, :, -1:], k, v)
    assert torch.allclose(o[:, :, 0], o_full[:, :, -1], atol=1e-5)
    assert torch.allclose(lse, l_full[:, :, -1], atol=1e-5)


def test_decode_fp64_loop():
    torch.manual_seed(42)
    B, Hq, Hkv, L, D = 2, 8, 4, 11, 16
    q = torch.randn(B, Hq, 1, D)
    k = torch.randn(B, Hkv, L, D)
    v = torch.randn(B, Hkv, L, D)
    o, lse = decode_attention(q, k, v)
    G = Hq // Hkv
    for b in range(B):
        for h in range(Hq):
            s = [sum(float(q[b, h, 0, d]) * float(k[b, h // G, j, d]) for d in range(D)) / math.sqrt(D)
                 for j in range(L)]
            m = max(s)
            z = sum(math.exp(x - m) for x in s)
            assert abs(float(lse[b, h]) - (m + math.log(z))) < 1e-5
            for d in range(D):
                ref = sum(math.exp(s[j] - m) / z * float(v[b, h // G, j, d]) for j in range(L))
                assert abs(float(o[b, h, 0, d]) - ref) < 1e-5


def test_single_kv_position_returns_v():
    q = torch.randn(1, 4, 1, 16)
    k = torch.randn(1, 2, 1, 16)
    v = torch.randn(1, 2, 1, 16)
    o, _ = decode_attention(q, k, v)
    assert torch.allclose(o[0, :, 0], v[0].repeat_interleave(2, 0)[:, 0], atol=1e-6)


def _reference_get_kv(pages, length):
    """The reference's get_kv: concat of pages 0, 1, ... taking `take` slots each."""
    chunks, remaining, i = [], length, 0
    while remaining > 0:
        take = min(pages.shape[2], remaining)
        chunks.append(pages[i, :, :take, :])
        remaining -= take
        i += 1
    return np.concatenate(chunks, axis=1)[None]


def test_gather_identity_table_matches_reference_get_kv():
    rng = np.random.default_rng(0)
    pages = rng.standard_normal((5, 3, 4, 6)).astype(np.float32)
    bt = np.arange(5, dtype=np.int32)[None]
    for length in (1, 3, 4, 7, 20):
        g = gather_pages(pages, bt, length)
        assert np.array_equal(g, _reference_get_kv(pages, length))


def test_gather_random_permutation_bruteforce():
    rng = np.random.default_rng(1)
    N, H, P, D = 12, 2, 4, 3
    pages = rng.integers(0, 1 << 15, size=(N, H, P, D)).astype(np.int16)
    perm = rng.permutation(N).astype(np.int32).reshape(3, 4)
    g = gather_pages(pages, perm, 13)
    for b in range(3):
        for h in range(H):
            for t in range(13):
                for d in range(D):
                    assert g[b, h, t, d] == pages[perm[b, t // P], h, t % P, d]


def test_gather_torch_is_bit_exact_for_bf16_and_nan():
    pages = torch.randn(6, 2, 4, 8).to(torch.bfloat16)
    pages[3, 1, 2, 5] = float("nan")
    bt = torch.tensor([[3, 0, 5]], dtype=torch.int32)
    g = gather_pages_torch(pages, bt, 12)
    raw = pages.view(torch.int16)
    for t in range(12):
        assert torch.equal(g[0, :, t].view(torch.int16), raw[int(bt[0, t // 4]), :, t % 4])


def test_merge_is_split_invariant():
    torch.manual_seed(7)
    q = torch.randn(1, 4, 1, 8)
    k = torch.randn(1, 2, 40, 8) * 2
    v = torch.randn(1, 2, 40, 8)
    o_ref, l_ref = decode_attention(q, k, v)
    for bounds in ([0, 40], [0, 13, 40], [0, 1, 2, 39, 40], list(range(0, 41, 8))):
        parts = [decode_attention(q, k[:, :, a:b], v[:, :, a:b]) for a, b in zip(bounds, bounds[1:])]
        o, lse = merge_splits(torch.stack([p[0][:, :, 0] for p in parts]),
                              torch.stack([p[1] for p in parts]))
        assert torch.allclose(o, o_ref[:, :, 0], atol=1e-5)
        assert torch.allclose(lse, l_ref, atol=1e-5)


def test_paged_decode_ragged_and_empty():
    torch.manual_seed(8)
    N, Hkv, P, D = 10, 2, 4, 8
    kp = torch.randn(N, Hkv, P, D)
    vp = torch.randn(N, Hkv, P, D)
    bt = torch.tensor([[7, 2, 9], [0, 5, 1], [4, 3, 6]], dtype=torch.int32)
    q = torch.randn(3, 4, 1, D)
    o, lse = paged_decode(q, kp, vp, bt, [5, 12, 0])
    for b, L in ((0, 5), (1, 12)):
        kk = torch.stack([kp[bt[b, t // P], :, t % P] for t in range(L)], 1)[None]
        vv = torch.stack([vp[bt[b, t // P], :, t % P] for t in range(L)], 1)[None]
        ob, lb = decode_attention(q[b:b + 1], kk, vv)
        assert torch.allclose(o[b], ob[0]) and torch.allclose(lse[b], lb[0])
    assert (o[2] == 0).all() and torch.isinf(lse[2]).all()


def test_decode_bias_equals_last_prefill_row_with_the_same_mask():
    """The decode oracle's additive mask matches the prefill oracle's on the last
    query row (the reference adds attention_mask the same way on both paths,
    models/llama3/attention.py:85-86)."""
    from oracle.attention import causal_attention

    g = torch.Generator().manual_seed(31)
    q = torch.randn(2, 8, 1, 16, generator=g)
    k = torch.randn(2, 2, 11, 16, generator=g)
    v = torch.randn(2, 2, 11, 16, generator=g)
    bias = 3.0 * torch.randn(2, 8, 11, generator=g)
    bias[0, :, 4] = float("-inf")
    o, lse = decode_attention(q, k, v, bias=bias)
    op, lp = causal_attention(q, k, v, q_offset=10, bias=bias.unsqueeze(2))
    assert torch.allclose(o, op, atol=1e-6) and torch.allclose(lse, lp[:, :, 0], atol=1e-6)


def test_paged_bias_shorter_than_the_sequence_is_zero_past_its_end():
    g = torch.Generator().manual_seed(32)
    P, lens = 4, [9, 3]
    kp = torch.randn(6, 1, P, 8, generator=g)
    vp = torch.randn(6, 1, P, 8, generator=g)
    bt = torch.tensor([[0, 2, 4], [1, -1, -1]], dtype=torch.int32)
    q = torch.randn(2, 2, 1, 8, generator=g)
    bias = torch.randn(2, 1, 5, generator=g)
    o, lse = paged_decode(q, kp, vp, bt, torch.tensor(lens), bias=bias)
    for b, L in enumerate(lens):
        kk = gather_pages_torch(kp, bt[b:b + 1], L)
        vv = gather_pages_torch(vp, bt[b:b + 1], L)
        full = torch.zeros(1, 2, L)
        n = min(L, 5)
        full[..., :n] = bias[b:b + 1, :, :n]
        r, rl = decode_attention(q[b:b + 1], kk, vv, bias=full)
        assert torch.allclose(o[b:b + 1], r) and torch.allclose(lse[b:b + 1], rl)
