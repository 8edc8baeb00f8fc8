"""Pins oracle.attention.causal_attention (prefill oracle) without retyping it.

Checks: an fp64 triple loop on tiny shapes (written as explicit per-element
sums, not matrix products), closed forms (row 0 returns v0; equal keys give
the prefix mean of V; S = 1), the lse invariant o = sum_j exp(s_j - lse) v_j,
GQA = per-head attention against kv head h // G, and q_offset equivalence
(the last rows of a longer prompt). The reference's own CPU parity test
(tests/test_triton_attention.py:37-47, seed 0, [2,4,8,16], atol 1e-5) is
reproduced against the brute force.

The additive mask (`bias`, the reference's attention_mask added to the scaled
scores, attention.py:457-477 and models/llama3/attention.py:85-86) is pinned
by the brute force with a bias term, the reference's own masked CPU case
(tests/test_triton_attention.py:78-90), and identities that hold whatever the
implementation: zero bias changes nothing, a per-row constant shifts only the
lse, ln 2 on a key equals that key appearing twice, -inf on keys equals
removing them, and a row whose visible keys all carry finfo.min averages them.
"""
import math

import pytest
import torch

from oracle.attention import causal_attention


def brute(q, k, v, q_offset=0, bias=None):
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = torch.zeros(B, Hq, Sq, D, dtype=torch.float64)
    lse = torch.full((B, Hq, Sq), float("-inf"), dtype=torch.float64)
    bias = None if bias is None else torch.broadcast_to(bias.double(), (B, Hq, Sq, Skv))
    for b in range(B):
        for h in range(Hq):
            kh = h // G
            for i in range(Sq):
                scores = []
                for j in range(Skv):
                    if j > i + q_offset:
                        break
                    s = 0.0
                    for d in range(D):
                        s += float(q[b, h, i, d]) * float(k[b, kh, j, d])
                    scores.append(s / math.sqrt(D) + (0.0 if bias is None else float(bias[b, h, i, j])))
                if not scores:
                    continue
                m = max(scores)
                z = sum(math.exp(s - m) for s in scores)
                lse[b, h, i] = m + math.log(z)
                for j, s in enumerate(scores):
                    w = math.exp(s - m) / z
                    for d in range(D):
                        out[b, h, i, d] += w * float(v[b, kh, j, d])
    return out, lse


@pytest.mark.parametrize("B,Hq,Hkv,S,D", [(1, 2, 2, 5, 4), (2, 4, 2, 6, 3), (1, 8, 2, 4, 8)])
def test_matches_bruteforce(B, Hq, Hkv, S, D):
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, Hq, S, D, generator=g)
    k = torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    o, lse = causal_attention(q, k, v)
    ob, lb = brute(q, k, v)
    assert torch.allclose(o.double(), ob, atol=1e-5)
    assert torch.allclose(lse.double(), lb, atol=1e-5)


def test_reference_cpu_parity_case():
    """tests/test_triton_attention.py:37-47 (seed 0, [2,4,8,16]) against brute force."""
    torch.manual_seed(0)
    q = torch.randn(2, 4, 8, 16)
    k = torch.randn(2, 4, 8, 16)
    v = torch.randn(2, 4, 8, 16)
    o, _ = causal_attention(q, k, v)
    ob, _ = brute(q, k, v)
    assert torch.allclose(o.double(), ob, atol=1e-5)


def test_row0_is_v0_and_single_token():
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 4, 7, 8, generator=g)
    k = torch.randn(2, 2, 7, 8, generator=g)
    v = torch.randn(2, 2, 7, 8, generator=g)
    o, lse = causal_attention(q, k, v)
    assert torch.allclose(o[:, 0::2, 0], v[:, :, 0], atol=1e-6)  # heads 0,2 -> kv 0,1
    assert torch.allclose(o[:, 1::2, 0], v[:, :, 0], atol=1e-6)
    # lse of row 0 is its only score
    s00 = (q[:, :, 0] * k.repeat_interleave(2, dim=1)[:, :, 0]).sum(-1) / math.sqrt(8)
    assert torch.allclose(lse[:, :, 0], s00, atol=1e-5)
    o1, _ = causal_attention(q[:, :, :1], k[:, :, :1], v[:, :, :1])
    assert torch.allclose(o1[:, :, 0], o[:, :, 0])


def test_equal_keys_give_prefix_mean():
    g = torch.Generator().manual_seed(3)
    S, D = 9, 4
    q = torch.randn(1, 2, S, D, generator=g)
    k = torch.randn(1, 1, 1, D, generator=g).expand(1, 1, S, D).contiguous()
    v = torch.randn(1, 1, S, D, generator=g)
    o, lse = causal_attention(q, k, v)
    prefix_mean = torch.cumsum(v[0, 0], 0) / torch.arange(1, S + 1).unsqueeze(1)
    assert torch.allclose(o[0, 0], prefix_mean, atol=1e-5)
    assert torch.allclose(o[0, 1], prefix_mean, atol=1e-5)
    # lse = s + log(i + 1) for equal scores s
    s = (q[0, :, :, :] * k[0, 0, 0]).sum(-1) / math.sqrt(D)
    assert torch.allclose(lse[0], s + torch.log(torch.arange(1, S + 1).float()), atol=1e-5)


def test_lse_invariant():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 4, 12, 8, generator=g) * 3
    k = torch.randn(1, 2, 12, 8, generator=g) * 3
    v = torch.randn(1, 2, 12, 8, generator=g)
    o, lse = causal_attention(q, k, v)
    kr = k.repeat_interleave(2, 1)
    vr = v.repeat_interleave(2, 1)
    s = torch.einsum("bhid,bhjd->bhij", q, kr) / math.sqrt(8)
    mask = torch.triu(torch.ones(12, 12, dtype=torch.bool), 1)
    w = torch.exp(s - lse.unsqueeze(-1)).masked_fill(mask, 0.0)
    assert torch.allclose(w.sum(-1), torch.ones(1, 4, 12), atol=1e-5)
    assert torch.allclose(torch.einsum("bhij,bhjd->bhid", w, vr), o, atol=1e-5)


def test_q_offset_equals_tail_of_full_prompt():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 4, 10, 8, generator=g)
    k = torch.randn(2, 2, 10, 8, generator=g)
    v = torch.randn(2, 2, 10, 8, generator=g)
    o_full, l_full = causal_attention(q, k, v)
    o_tail, l_tail = causal_attention(q[:, :, 7:], k, v, q_offset=7)
    assert torch.allclose(o_tail, o_full[:, :, 7:], atol=1e-6)
    assert torch.allclose(l_tail, l_full[:, :, 7:], atol=1e-6)
    ob, lb = brute(q[:, :, 7:], k, v, q_offset=7)
    assert torch.allclose(o_tail.double(), ob, atol=1e-5)


def test_row_chunking_is_invisible():
    g = torch.Generator().manual_seed(6)
    q = torch.randn(1, 2, 37, 8, generator=g)
    k = torch.randn(1, 1, 37, 8, generator=g)
    v = torch.randn(1, 1, 37, 8, generator=g)
    a, la = causal_attention(q, k, v, row_chunk=5)
    b, lb = causal_attention(q, k, v)
    assert torch.allclose(a, b, atol=1e-6) and torch.allclose(la, lb, atol=1e-6)


def test_empty_keys_give_zero_and_neg_inf():
    q = torch.randn(1, 2, 3, 4)
    k = torch.zeros(1, 1, 0, 4)
    o, lse = causal_attention(q, k, k)
    assert (o == 0).all() and torch.isinf(lse).all() and (lse < 0).all()


def _autograd_reference(q, k, v, do, q_offset=0):
    """Independent path: torch autograd through a dense fp64 masked softmax."""
    G = q.shape[1] // k.shape[1]
    qd, kd, vd = (t.double().clone().requires_grad_(True) for t in (q, k, v))
    kr = kd.repeat_interleave(G, dim=1)
    vr = vd.repeat_interleave(G, dim=1)
    s = qd @ kr.transpose(-1, -2) / math.sqrt(q.shape[-1])
    Sq, Skv = q.shape[2], k.shape[2]
    mask = torch.arange(Skv).view(1, Skv) > (torch.arange(Sq).view(Sq, 1) + q_offset)
    s = s.masked_fill(mask, float("-inf"))
    o = torch.softmax(s, -1) @ vr
    (o * do.double()).sum().backward()
    return qd.grad, kd.grad, vd.grad


@pytest.mark.parametrize("B,Hq,Hkv,S,D,off", [(1, 2, 2, 5, 4, 0), (2, 4, 2, 9, 8, 0),
                                              (1, 4, 1, 7, 16, 3), (2, 3, 3, 16, 32, 0)])
def test_backward_matches_fp64_autograd(B, Hq, Hkv, S, D, off):
    from oracle.attention import causal_attention_backward

    g = torch.Generator().manual_seed(S * 10 + D)
    q = torch.randn(B, Hq, S, D, generator=g)
    k = torch.randn(B, Hkv, S + off, D, generator=g)
    v = torch.randn(B, Hkv, S + off, D, generator=g)
    do = torch.randn(B, Hq, S, D, generator=g)
    got = causal_attention_backward(q, k, v, do, q_offset=off, row_chunk=4)
    ref = _autograd_reference(q, k, v, do, q_offset=off)
    for gt, rf in zip(got, ref):
        assert (gt.double() - rf).abs().max().item() < 1e-5


def test_backward_matches_finite_differences():
    """dq, dk, dv against central differences of sum(O * dO) in fp64 (tiny shape)."""
    from oracle.attention import causal_attention, causal_attention_backward

    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 4, 3, generator=g, dtype=torch.float64)
    k = torch.randn(1, 1, 4, 3, generator=g, dtype=torch.float64)
    v = torch.randn(1, 1, 4, 3, generator=g, dtype=torch.float64)
    do = torch.randn(1, 2, 4, 3, generator=g, dtype=torch.float64)

    def loss(qq, kk, vv):
        o, _ = causal_attention(qq, kk, vv)
        return (o.double() * do).sum().item()

    dq, dk, dv = causal_attention_backward(q, k, v, do)
    eps = 1e-4
    for t, grad in ((q, dq), (k, dk), (v, dv)):
        for idx in [(0, 0, 0, 0), (0, 0, 3, 2), (0, t.shape[1] - 1, 2, 1)]:
            tp, tm = t.clone(), t.clone()
            tp[idx] += eps
            tm[idx] -= eps
            args_p = [tp if x is t else x for x in (q, k, v)]
            args_m = [tm if x is t else x for x in (q, k, v)]
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            assert abs(fd - grad[idx].item()) < 2e-3 * max(1.0, abs(fd))


def test_backward_of_fully_masked_rows_is_zero():
    """With Skv = 0 nothing is visible: every gradient is zero (no NaN)."""
    from oracle.attention import causal_attention_backward

    q = torch.randn(1, 2, 3, 8)
    kv = torch.zeros(1, 1, 0, 8)
    dq, dk, dv = causal_attention_backward(q, kv, kv, torch.randn(1, 2, 3, 8))
    assert torch.equal(dq, torch.zeros_like(dq)) and dk.numel() == 0 and dv.numel() == 0


# ---------------------------------------------------------------------------
# additive mask (bias)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", ["key", "rows", "full"])
def test_bias_matches_bruteforce(shape):
    g = torch.Generator().manual_seed(21)
    B, Hq, Hkv, S, D = 2, 4, 2, 6, 4
    q = torch.randn(B, Hq, S, D, generator=g)
    k = torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    dims = {"key": (B, 1, 1, S), "rows": (1, 1, S, S), "full": (B, Hq, S, S)}[shape]
    bias = 2.0 * torch.randn(*dims, generator=g)
    o, lse = causal_attention(q, k, v, bias=bias)
    ob, lb = brute(q, k, v, bias=bias)
    assert torch.allclose(o.double(), ob, atol=1e-5)
    assert torch.allclose(lse.double(), lb, atol=1e-5)


def test_reference_masked_cpu_case():
    """tests/test_triton_attention.py:78-90: seed 1, [1, 2, 6, 8] fp32, a key mask
    [1, 1, 1, 6] of -1e4 on the last two keys, atol/rtol 1e-5."""
    torch.manual_seed(1)
    q = torch.randn(1, 2, 6, 8)
    k = torch.randn(1, 2, 6, 8)
    v = torch.randn(1, 2, 6, 8)
    mask = torch.zeros((1, 1, 1, 6))
    mask[..., -2:] = -1e4
    o, _ = causal_attention(q, k, v, bias=mask)
    ob, _ = brute(q, k, v, bias=mask)
    assert torch.allclose(o.double(), ob, atol=1e-5, rtol=1e-5)
    # rows 0..3 never see the masked keys: unchanged by the mask
    o0, _ = causal_attention(q, k, v)
    assert torch.equal(o[:, :, :4], o0[:, :, :4])


def test_zero_bias_changes_nothing_and_row_constants_shift_lse():
    g = torch.Generator().manual_seed(22)
    q = torch.randn(1, 4, 9, 8, generator=g)
    k = torch.randn(1, 2, 9, 8, generator=g)
    v = torch.randn(1, 2, 9, 8, generator=g)
    o0, l0 = causal_attention(q, k, v)
    o1, l1 = causal_attention(q, k, v, bias=torch.zeros(1, 1, 9, 9))
    assert torch.equal(o0, o1) and torch.equal(l0, l1)
    c = 5.0 * torch.randn(1, 4, 9, 1, generator=g)
    o2, l2 = causal_attention(q, k, v, bias=c.expand(1, 4, 9, 9))
    assert torch.allclose(o2, o0, atol=1e-5)
    assert torch.allclose(l2, l0 + c[..., 0], atol=1e-5)


def test_ln2_bias_equals_a_duplicated_key():
    """softmax(s + ln 2 on key j) weighs key j as if it appeared twice (every key
    visible: q_offset >= Skv)."""
    g = torch.Generator().manual_seed(23)
    Skv, j = 7, 3
    q = torch.randn(1, 2, 4, 8, generator=g)
    k = torch.randn(1, 1, Skv, 8, generator=g)
    v = torch.randn(1, 1, Skv, 8, generator=g)
    bias = torch.zeros(1, 1, 1, Skv)
    bias[..., j] = math.log(2.0)
    o, lse = causal_attention(q, k, v, q_offset=Skv, bias=bias)
    kd = torch.cat([k, k[:, :, j:j + 1]], dim=2)
    vd = torch.cat([v, v[:, :, j:j + 1]], dim=2)
    od, ld = causal_attention(q, kd, vd, q_offset=Skv + 1)
    assert torch.allclose(o, od, atol=1e-5) and torch.allclose(lse, ld, atol=1e-5)


def test_neg_inf_bias_equals_removed_keys():
    g = torch.Generator().manual_seed(24)
    q = torch.randn(2, 2, 5, 8, generator=g)
    k = torch.randn(2, 2, 8, 8, generator=g)
    v = torch.randn(2, 2, 8, 8, generator=g)
    bias = torch.zeros(2, 1, 1, 8)
    bias[..., 5:] = float("-inf")
    o, lse = causal_attention(q, k, v, q_offset=8, bias=bias)
    ot, lt = causal_attention(q, k[:, :, :5], v[:, :, :5], q_offset=8)
    assert torch.allclose(o, ot, atol=1e-6) and torch.allclose(lse, lt, atol=1e-6)
    # every key at -inf: no finite score, o = 0 and lse = -inf
    o, lse = causal_attention(q, k, v, bias=torch.full((1, 1, 1, 8), float("-inf")))
    assert (o == 0).all() and torch.isinf(lse).all()


def test_finfo_min_rows_average_their_visible_keys():
    """A padded query row whose visible keys all carry finfo.min (the usual
    padding mask) gets the uniform average of those keys, as torch.softmax of
    equal scores gives in the reference."""
    g = torch.Generator().manual_seed(25)
    q = torch.randn(1, 1, 6, 4, generator=g)
    k = torch.randn(1, 1, 6, 4, generator=g)
    v = torch.randn(1, 1, 6, 4, generator=g)
    bias = torch.zeros(1, 1, 6, 6)
    bias[:, :, :3, :] = torch.finfo(torch.float32).min   # rows 0..2: every key masked
    o, _ = causal_attention(q, k, v, bias=bias)
    for i in range(3):
        assert torch.allclose(o[0, 0, i], v[0, 0, :i + 1].mean(0), atol=1e-6)


def test_backward_with_bias_matches_fp64_autograd():
    from oracle.attention import causal_attention_backward

    g = torch.Generator().manual_seed(26)
    q = torch.randn(2, 4, 7, 8, generator=g)
    k = torch.randn(2, 2, 9, 8, generator=g)
    v = torch.randn(2, 2, 9, 8, generator=g)
    do = torch.randn(2, 4, 7, 8, generator=g)
    bias = 1.5 * torch.randn(2, 1, 7, 9, generator=g)
    bias[1, :, :, 0] = -1e4
    got = causal_attention_backward(q, k, v, do, q_offset=2, bias=bias, row_chunk=3)
    G = 2
    qd, kd, vd = (t.double().clone().requires_grad_(True) for t in (q, k, v))
    s = qd @ kd.repeat_interleave(G, 1).transpose(-1, -2) / math.sqrt(8) + bias.double()
    mask = torch.arange(9).view(1, 9) > (torch.arange(7).view(7, 1) + 2)
    o = torch.softmax(s.masked_fill(mask, float("-inf")), -1) @ vd.repeat_interleave(G, 1)
    (o * do.double()).sum().backward()
    for gt, rf in zip(got, (qd.grad, kd.grad, vd.grad)):
        assert (gt.double() - rf).abs().max().item() < 1e-5
