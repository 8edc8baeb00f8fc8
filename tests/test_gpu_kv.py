"""GPU bit-exactness of the page-pool append and gather kernels.

Identity table: the gathered cache equals the reference's get_kv (concat of
pages, models/llama3/kv_cache.py:65-83) and the appended tokens
(test_llama3_shapes.py:130-149 round trip). Random permutation tables equal
the numpy gather of the oracle, element for element (compared as raw bits).
"""
import numpy as np
import pytest
import torch

from oracle.decode import gather_pages

pytestmark = pytest.mark.gpu


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_append_get_round_trip_identity_table(cuda, dtype):
    from llm_cuda.models.llama3.kv_cache import PagedKVLayerCache

    cache = PagedKVLayerCache(4, 8, 16, 4, cuda, dtype)
    k = torch.randn(1, 4, 6, 8, device=cuda).to(dtype)
    v = torch.randn(1, 4, 6, 8, device=cuda).to(dtype)
    cache.append(k, v)
    ko, vo = cache.get_kv()
    assert cache.length == 6 and ko.shape == (1, 4, 6, 8)
    assert torch.equal(_bits(ko), _bits(k)) and torch.equal(_bits(vo), _bits(v))
    # token t sits in physical page t // 4, slot t % 4 (identity mapping)
    for t in range(6):
        assert torch.equal(_bits(cache.key_pages[t // 4, :, t % 4]), _bits(k[0, :, t]))
    k2 = torch.randn(1, 4, 1, 8, device=cuda).to(dtype)
    cache.append(k2, k2)
    ko, _ = cache.get_kv()
    assert torch.equal(_bits(ko[:, :, 6]), _bits(k2[:, :, 0]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("P", [64, 5])
def test_batched_append_random_permutation(cuda, dtype, P):
    from llm_cuda.kernels import _ops

    g = torch.Generator().manual_seed(P)
    B, H, D, maxp = 3, 2, 64, 6
    N = B * maxp + 2
    perm = torch.randperm(N, generator=g)[: B * maxp].to(torch.int32).view(B, maxp)
    kp = torch.zeros(N, H, P, D, dtype=dtype, device=cuda)
    vp = torch.zeros_like(kp)
    start = torch.tensor([0, 7, P * 2 - 1], dtype=torch.int32)
    S = P + 3
    kn = torch.randn(B, S, H, D, generator=g).to(dtype).transpose(1, 2)  # strided view
    vn = torch.randn(B, S, H, D, generator=g).to(dtype).transpose(1, 2)
    _ops.kv_append(kn.to(cuda), vn.to(cuda), kp, vp, perm.to(cuda), start.to(cuda))
    kp_c, bt = kp.cpu(), perm.numpy()
    for b in range(B):
        for s in range(S):
            t = int(start[b]) + s
            page = bt[b, t // P]
            assert torch.equal(_bits(kp_c[page, :, t % P]), _bits(kn[b, :, s]))
    # gather through the same table == numpy oracle, bit for bit
    L = int(start.min()) + S
    ko, vo = _ops.kv_gather(kp, vp, perm.to(cuda), L)
    expect = gather_pages(_bits(kp_c).numpy(), bt, L)
    assert np.array_equal(_bits(ko).numpy(), expect)
    assert np.array_equal(_bits(vo).numpy(), gather_pages(_bits(vp.cpu()).numpy(), bt, L))


def test_append_drops_tokens_beyond_capacity_or_bad_pages(cuda):
    from llm_cuda.kernels import _ops

    kp = torch.zeros(4, 1, 4, 8, device=cuda)
    vp = torch.zeros_like(kp)
    bt = torch.tensor([[0, -1], [2, 99]], dtype=torch.int32, device=cuda)
    start = torch.tensor([2, 6], dtype=torch.int32, device=cuda)
    kn = torch.ones(2, 1, 4, 8, device=cuda)
    _ops.kv_append(kn, kn, kp, vp, bt, start)
    kc = kp.cpu()
    assert (kc[0, 0, 2:] == 1).all() and (kc[0, 0, :2] == 0).all()  # seq 0: t=2,3 kept; 4,5 -> page -1
    assert (kc[1] == 0).all() and (kc[3] == 0).all()              # nothing else written
    assert (kc[2] == 0).all()                                     # seq 1 starts in page 99 / beyond


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,D,Hq,Hkv", [(1, 64, 4, 2), (3, 128, 4, 2), (2, 20, 4, 2),
                                         (5, 128, 32, 8)])
def test_rope_kv_append_equals_rope_then_append(cuda, dtype, S, D, Hq, Hkv):
    """The fused decode-time op equals the RoPE kernel followed by the page
    append and the length update, bit for bit: rotated q, both pools (with a
    ragged batch, an invalid page entry and strided projection views) and the
    advanced seq_lens. D = 20 takes the element-wise path; the 32/8-head case
    has more items per sequence than one workgroup's 1024 threads."""
    from llm_cuda.kernels import _ops
    from llm_cuda.models.llama3.rotary import build_rope_cache

    g = torch.Generator().manual_seed(S * 100 + D + Hq)
    B, P, maxp = 3, 8, 5
    N = B * maxp + 1
    table = torch.randperm(N, generator=g)[: B * maxp].to(torch.int32).view(B, maxp)
    table[2, 3] = -1  # sequence 2: its 4th page is unmapped (tokens dropped)
    table = table.to(cuda)
    lens = torch.tensor([0, 7, 23], dtype=torch.int32, device=cuda)
    pools = [torch.randn(N, Hkv, P, D, generator=g).to(dtype).to(cuda) for _ in range(2)]
    qkv = torch.randn(B, S, (Hq + 2 * Hkv) * D, generator=g).to(dtype).to(cuda)
    q = qkv[..., :Hq * D].view(B, S, Hq, D).transpose(1, 2)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].view(B, S, Hkv, D).transpose(1, 2)
    v = qkv[..., (Hq + Hkv) * D:].view(B, S, Hkv, D).transpose(1, 2)
    cos, sin = build_rope_cache(maxp * P, D, 10000.0, torch.device(cuda), dtype)

    # separate kernels: per-sequence positions, so rotate each sequence alone
    ref_k, ref_v = pools[0].clone(), pools[1].clone()
    ref_q = torch.empty(B, Hq, S, D, dtype=dtype, device=cuda)
    for b in range(B):
        p0 = int(lens[b])
        qb, kb = _ops.rope(q[b:b + 1], cos[p0:p0 + S], sin[p0:p0 + S], k[b:b + 1])
        ref_q[b] = qb[0]
        _ops.kv_append(kb, v[b:b + 1], ref_k, ref_v, table[b:b + 1], lens[b:b + 1].clone())
    got_k, got_v = pools[0].clone(), pools[1].clone()
    got_lens = lens.clone()
    got_q = _ops.rope_kv_append(q, k, v, cos, sin, got_k, got_v, table, got_lens)
    assert torch.equal(_bits(got_q), _bits(ref_q))
    assert torch.equal(_bits(got_k), _bits(ref_k)) and torch.equal(_bits(got_v), _bits(ref_v))
    assert torch.equal(got_lens.cpu(), (lens + S).cpu())


def test_rope_kv_append_rejects_short_tables(cuda):
    from llm_cuda.kernels import _ops

    B, H, D, P, maxp = 1, 2, 64, 8, 4
    pools = [torch.zeros(maxp, H, P, D, device=cuda) for _ in range(2)]
    table = torch.arange(maxp, dtype=torch.int32, device=cuda).view(1, maxp)
    x = torch.zeros(B, H, 1, D, device=cuda)
    cos = torch.zeros(maxp * P - 1, D, device=cuda)
    with pytest.raises(RuntimeError, match="cover the block-table capacity"):
        _ops.rope_kv_append(x, x, x, cos, cos, pools[0], pools[1], table,
                            torch.zeros(1, dtype=torch.int32, device=cuda))
