"""GPU parity of the fused decode step (lc_paged_decode_step): RoPE of the new
token at p = seq_lens[b], its append to the page pools and decode attention
over the cache including it, in one launch.

The oracle is the unfused sequence this build already pins: rope_kv_append
(bit-exact against the RoPE kernel followed by the page append) and the oracle's
paged decode over the advanced lengths. The pools and lengths after the fused
step must equal the unfused ones bit for bit; out and lse match the oracle to the
decode tolerances. Cases: ragged positions including an empty sequence, a page
boundary, the last slot of the capacity, a position past the capacity and a
position whose page entry is invalid (both dropped); two head groups (G = 20);
head_dim 64 and 256; masks; several steps in a row; graph replays.
"""
import pytest
import torch

from helpers import ATOL, assert_close, assert_lse_close
from oracle.decode import paged_decode

pytestmark = pytest.mark.gpu


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def _case(lens, Hq, Hkv, D, P, maxp, dtype, device, seed):
    from llm_cuda.models.llama3.rotary import build_rope_cache

    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    N = B * maxp + 2
    table = torch.randperm(N, generator=g)[: B * maxp].to(torch.int32).view(B, maxp)
    pools = [torch.randn(N, Hkv, P, D, generator=g).to(dtype) for _ in range(2)]
    qkv = torch.randn(B, 1, (Hq + 2 * Hkv) * D, generator=g).to(dtype)
    q = qkv[..., :Hq * D].view(B, 1, Hq, D).transpose(1, 2)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].view(B, 1, Hkv, D).transpose(1, 2)
    v = qkv[..., (Hq + Hkv) * D:].view(B, 1, Hkv, D).transpose(1, 2)
    cos, sin = build_rope_cache(maxp * P, D, 500000.0, torch.device("cpu"), dtype)
    lens = torch.tensor(lens, dtype=torch.int32)
    to = lambda t: t.to(device)  # noqa: E731
    return (to(q), to(k), to(v), to(cos), to(sin), to(pools[0]), to(pools[1]), to(table),
            to(lens))


def _unfused(q, k, v, cos, sin, kp, vp, table, lens, mask=None):
    """rope_kv_append, then the oracle's decode over the advanced lengths."""
    from llm_cuda.kernels import _ops

    kp, vp, lens = kp.clone(), vp.clone(), lens.clone()
    q_rot = _ops.rope_kv_append(q, k, v, cos, sin, kp, vp, table, lens)
    bias = None if mask is None else mask[:, :, 0].cpu()
    cap = table.shape[1] * kp.shape[2]  # the kernels clamp lengths to the capacity
    ref, ref_lse = paged_decode(q_rot.cpu(), kp.cpu(), vp.cpu(), table.cpu(),
                                lens.cpu().clamp(0, cap), bias=bias)
    return ref, ref_lse, kp, vp, lens


def _fused(q, k, v, cos, sin, kp, vp, table, lens, mask=None):
    from llm_cuda.kernels import _ops

    kp, vp, lens = kp.clone(), vp.clone(), lens.clone()
    counters = torch.zeros_like(lens)
    out, lse = _ops.paged_decode_step(q, k, v, cos, sin, kp, vp, table, lens, counters,
                                      attention_mask=mask, return_lse=True)
    assert (counters.cpu() == 0).all(), "the step must leave its counters at zero"
    return out, lse, kp, vp, lens


def _check(fused, unfused, dtype, what):
    out, lse, kp, vp, lens = fused
    ref, ref_lse, rkp, rvp, rlens = unfused
    assert torch.equal(lens.cpu(), rlens.cpu()), f"{what}: lengths"
    assert torch.equal(_bits(kp), _bits(rkp)) and torch.equal(_bits(vp), _bits(rvp)), \
        f"{what}: pools differ from RoPE + append"
    assert_close(out, ref, ATOL[dtype], what)
    assert_lse_close(lse, ref_lse, what)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (40, 2, 128), (16, 4, 64), (8, 2, 256)])
def test_decode_step_equals_rope_append_then_decode(cuda, dtype, Hq, Hkv, D):
    P, maxp = 64, 6  # capacity 384
    # p = 0 (empty cache), 63 / 64 (page boundary), ragged, 383 (the last
    # slot), 384 and 1000 (past the capacity: dropped, the cache is attended)
    lens = [0, 63, 64, 200, 383, 384, 1000, 129]
    case = _case(lens, Hq, Hkv, D, P, maxp, dtype, cuda, seed=Hq + D)
    _check(_fused(*case), _unfused(*case), dtype, f"step Hq={Hq} Hkv={Hkv} D={D}")


def test_decode_step_invalid_page_at_the_new_position(cuda):
    """The new token's page entry is invalid: it is neither written nor
    attended. The reference here is rope_kv_append followed by the split-K
    decode kernel (whose skipping of invalid pages is pinned against the
    oracle in the decode tests)."""
    from llm_cuda.kernels import _ops

    dtype = torch.bfloat16
    q, k, v, cos, sin, kp, vp, table, lens = _case([130, 70], 16, 4, 128, 64, 4, dtype, cuda,
                                                   seed=7)
    table[0, 2] = -1  # position 130 lives in page 2
    table[1, 1] = 10 ** 6  # positions 64 .. 70 live in page 1
    out, lse, f_kp, f_vp, f_lens = _fused(q, k, v, cos, sin, kp, vp, table, lens)
    u_kp, u_vp, u_lens = kp.clone(), vp.clone(), lens.clone()
    q_rot = _ops.rope_kv_append(q, k, v, cos, sin, u_kp, u_vp, table, u_lens)
    ref, ref_lse = _ops.paged_decode(q_rot, u_kp, u_vp, table, u_lens, return_lse=True,
                                     split_tokens=64)
    assert torch.equal(f_lens.cpu(), u_lens.cpu()) and torch.equal(_bits(f_kp), _bits(u_kp))
    assert torch.equal(_bits(f_vp), _bits(u_vp))
    assert_close(out, ref, ATOL[dtype], "invalid page")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("per_head", [False, True])
def test_decode_step_with_mask(cuda, per_head):
    """An additive mask over tokens 0 .. p (shorter than some positions, with
    -inf and large negative entries), the new token's own entry included."""
    dtype = torch.bfloat16
    lens = [100, 5, 300, 64]
    Hq, Hkv, D = 16, 4, 128
    case = _case(lens, Hq, Hkv, D, 64, 6, dtype, cuda, seed=11 + int(per_head))
    g = torch.Generator().manual_seed(3)
    L = 200
    mask = torch.randn(len(lens), Hq if per_head else 1, 1, L, generator=g)
    mask[0, ..., 100] = float("-inf")  # sequence 0's new token (p = 100) masked out
    mask[2, ..., :20] = -1e4
    mask[1, ..., 5] = 3.0  # sequence 1's new token boosted
    mask = mask.to(cuda)
    _check(_fused(*case, mask=mask), _unfused(*case, mask=mask), dtype,
           f"masked step per_head={per_head}")


def test_decode_steps_in_a_row_and_graph_replays(cuda):
    """Three fused steps in a row equal three unfused steps (each new token is
    cached for the next); then one captured step replayed three times, with
    eager work between the replays, equals the eager sequence every time."""
    from llm_cuda.kernels import _ops

    dtype = torch.bfloat16
    Hq, Hkv, D, P, maxp = 32, 8, 128, 64, 5
    lens0 = [17, 64, 250, 0]
    q, k, v, cos, sin, kp, vp, table, lens = _case(lens0, Hq, Hkv, D, P, maxp, dtype, cuda,
                                                   seed=23)
    g = torch.Generator().manual_seed(5)
    news = [[torch.randn(t.shape, generator=g).to(dtype).to(cuda) for t in (q, k, v)]
            for _ in range(6)]
    f_kp, f_vp, f_lens = kp.clone(), vp.clone(), lens.clone()
    u_kp, u_vp, u_lens = kp.clone(), vp.clone(), lens.clone()
    counters = torch.zeros_like(lens)
    for step in range(3):
        qs, ks, vs = news[step]
        out = _ops.paged_decode_step(qs, ks, vs, cos, sin, f_kp, f_vp, table, f_lens, counters)
        q_rot = _ops.rope_kv_append(qs, ks, vs, cos, sin, u_kp, u_vp, table, u_lens)
        ref, _ = paged_decode(q_rot.cpu(), u_kp.cpu(), u_vp.cpu(), table.cpu(), u_lens.cpu())
        assert_close(out, ref, ATOL[dtype], f"step {step}")
        assert torch.equal(_bits(f_kp), _bits(u_kp)) and torch.equal(f_lens.cpu(), u_lens.cpu())

    # graph: static inputs, one captured step, replays advance the lengths
    sq, sk, sv = (t.clone() for t in news[3])
    static_out = torch.empty(len(lens0), Hq, 1, D, dtype=dtype, device=cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    warm_kp, warm_vp, warm_lens = f_kp.clone(), f_vp.clone(), f_lens.clone()
    with torch.cuda.stream(s):  # warm-up on copies, so the captured state is untouched
        _ops.paged_decode_step(sq, sk, sv, cos, sin, warm_kp, warm_vp, table, warm_lens, counters)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o = _ops.paged_decode_step(sq, sk, sv, cos, sin, f_kp, f_vp, table, f_lens, counters)
        static_out.copy_(o)
    for rep in range(3):
        qs, ks, vs = news[3 + rep]
        sq.copy_(qs)
        sk.copy_(ks)
        sv.copy_(vs)
        graph.replay()
        torch.cuda.synchronize()
        q_rot = _ops.rope_kv_append(qs, ks, vs, cos, sin, u_kp, u_vp, table, u_lens)
        ref, _ = paged_decode(q_rot.cpu(), u_kp.cpu(), u_vp.cpu(), table.cpu(), u_lens.cpu())
        assert_close(static_out, ref, ATOL[dtype], f"replay {rep}")
        assert torch.equal(_bits(f_kp), _bits(u_kp)) and torch.equal(f_lens.cpu(), u_lens.cpu())
        assert (counters.cpu() == 0).all()
        torch.cuda.synchronize()


def test_decode_step_rejects_what_it_cannot_run(cuda):
    from llm_cuda.kernels import _ops

    dtype = torch.bfloat16
    q, k, v, cos, sin, kp, vp, table, lens = _case([3], 8, 2, 128, 64, 2, dtype, cuda, seed=1)
    counters = torch.zeros_like(lens)
    with pytest.raises(ValueError, match="fused decode step"):  # fp32
        _ops.paged_decode_step(q.float(), k.float(), v.float(), cos.float(), sin.float(),
                               kp.float(), vp.float(), table, lens, counters)
    with pytest.raises(RuntimeError, match="cover the block-table capacity"):
        _ops.paged_decode_step(q, k, v, cos[:100], sin[:100], kp, vp, table, lens, counters)
