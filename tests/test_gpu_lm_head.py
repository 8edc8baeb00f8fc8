"""GPU parity: fused lm_head + greedy argmax vs the oracle (oracle/lm_head.py).

The ids are an index derived from floating-point logits. The GPU sums each dot
product in fp32 in its own order, so a logit that sits on a rounding boundary
of the model dtype may round one ulp away from the oracle's fp64 sum. The bar:
identical ids, except that where they differ the two candidates' exact (fp64)
logits must lie within one ulp of the model dtype of each other; the number of
such rows is also bounded. The winning logit must equal the oracle's rounded
logit at the returned id.
"""
import pytest
import torch

from oracle.lm_head import lm_head_argmax as oracle_argmax

pytestmark = pytest.mark.gpu

# Relative spacing of the model dtype (bf16, f16); for fp32 logits, the
# accumulated rounding of a K-term fp32 sum in another order (K <= 4096).
ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 1e-5}


def _check(hidden, weight, max_mismatch=0):
    from llm_cuda.kernels import _ops

    ids, best = _ops.lm_head_argmax(hidden, weight, return_max=True)
    assert ids.dtype == torch.int64 and ids.shape == (hidden.shape[0],)
    ref_ids, _, ref_logits = oracle_argmax(hidden, weight)
    ids_c = ids.cpu()
    h64 = hidden.detach().cpu().double()
    w64 = weight.detach().cpu().double()
    mism = (ids_c != ref_ids).nonzero().view(-1).tolist()
    assert len(mism) <= max_mismatch, f"{len(mism)} rows differ: {mism[:8]}"
    for b in mism:
        a, r = int(ids_c[b]), int(ref_ids[b])
        la = float(h64[b] @ w64[a])
        lr = float(h64[b] @ w64[r])
        tol = ULP[hidden.dtype] * max(abs(lr), 2.0 ** -20)
        assert abs(la - lr) <= tol, f"row {b}: id {a} ({la}) vs oracle {r} ({lr})"
    # The winning logit is the rounded logit at the returned id (up to the same
    # rounding-boundary slack).
    got = ref_logits.float().gather(-1, ids_c.view(-1, 1)).view(-1)
    slack = ULP[hidden.dtype] * got.abs().clamp(min=2.0 ** -20)
    assert ((best.cpu() - got).abs() <= slack).all()


@pytest.mark.parametrize("B,K,V,dtype", [
    (1, 128, 1000, torch.bfloat16),        # one tile, partial last vocab block
    (5, 256, 4099, torch.bfloat16),
    (32, 512, 12800, torch.float16),
    (33, 384, 3000, torch.bfloat16),       # two batch chunks on the MFMA path
    (70, 128, 515, torch.bfloat16),
    (3, 200, 777, torch.bfloat16),         # K % 128 != 0: generic kernel
    (2, 256, 32000, torch.float32),        # config 1 (tiny Llama-3, fp32)
])
def test_lm_head_argmax_matches_oracle(cuda, B, K, V, dtype):
    g = torch.Generator().manual_seed(B * 7 + K)
    hidden = torch.randn(B, K, generator=g).to(dtype).to(cuda)
    weight = (torch.randn(V, K, generator=g) * 0.02).to(dtype).to(cuda)
    _check(hidden, weight)


def test_lm_head_argmax_config4_shape(cuda):
    """Llama-3-8B lm_head (vocab 128256, hidden 4096, bf16), batch 32; weights
    ~N(0, 0.02) as the model's initialiser, hidden states ~N(0, 1)."""
    g = torch.Generator(device=cuda).manual_seed(0)
    hidden = torch.randn(32, 4096, generator=g, device=cuda).bfloat16()
    weight = (torch.randn(128256, 4096, generator=g, device=cuda) * 0.02).bfloat16()
    _check(hidden, weight, max_mismatch=1)


def test_lm_head_argmax_strided_last_position(cuda):
    """hidden_states[:, -1, :] of a [B, S, K] tensor (row stride S*K)."""
    g = torch.Generator().manual_seed(4)
    hs = torch.randn(6, 9, 256, generator=g).bfloat16().to(cuda)
    weight = (torch.randn(2000, 256, generator=g) * 0.02).bfloat16().to(cuda)
    _check(hs[:, -1, :], weight)


def test_lm_head_argmax_ties_and_nan(cuda):
    from llm_cuda.kernels import _ops

    g = torch.Generator().manual_seed(9)
    K, V = 256, 1000
    hidden = torch.randn(4, K, generator=g).bfloat16()
    weight = (torch.randn(V, K, generator=g) * 0.02).bfloat16()
    winner = oracle_argmax(hidden, weight)[0]
    # copies of each row's winner at other indices, across workgroup boundaries:
    # equal logits, so the smallest index of each group must win
    for b in range(4):
        weight[900 - b] = weight[winner[b]]
        weight[130 + b] = weight[winner[b]]
    expect = oracle_argmax(hidden, weight)[0]
    assert all(expect[b] <= min(int(winner[b]), 130 + b) for b in range(4))
    ids = _ops.lm_head_argmax(hidden.to(cuda), weight.to(cuda)).cpu()
    assert torch.equal(ids, expect)
    # NaN in a weight row: every batch row picks the first NaN row
    weight[777] = float("nan")
    weight[300, 5] = float("nan")
    ids = _ops.lm_head_argmax(hidden.to(cuda), weight.to(cuda)).cpu()
    assert ids.tolist() == [300] * 4


def test_lm_head_argmax_rejects_bad_shapes(cuda):
    from llm_cuda.kernels import _ops

    h = torch.zeros(2, 128, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        _ops.lm_head_argmax(h, torch.zeros(10, 64, device=cuda, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        _ops.lm_head_argmax(h, torch.zeros(10, 128, device=cuda, dtype=torch.float16))


def _abi_call(hidden, weight, counters):
    from llm_cuda import _native

    lib = _native.load()
    B, K = hidden.shape
    V = weight.shape[0]
    ids = torch.full((B,), -7, dtype=torch.int64, device=hidden.device)
    mx = torch.full((B,), float("nan"), dtype=torch.float32, device=hidden.device)
    ws = torch.empty(max(lib.lc_lm_head_argmax_workspace_bytes(B, V), 16), dtype=torch.uint8,
                     device=hidden.device)
    rc = lib.lc_lm_head_argmax(hidden.data_ptr(), hidden.stride(0), weight.data_ptr(),
                               weight.stride(0), B, K, V, ids.data_ptr(), mx.data_ptr(),
                               ws.data_ptr(), ws.numel(),
                               None if counters is None else counters.data_ptr(),
                               _native.lc_dtype(hidden), torch.cuda.current_stream().cuda_stream)
    _native.check(rc, "lc_lm_head_argmax")
    return ids, mx


@pytest.mark.parametrize("B,K,V", [(1, 128, 10), (32, 4096, 20000), (33, 512, 3000),
                                   (7, 256, 16385), (4, 1024, 64),
                                   (32, 512, 60000),    # block pool: 3 blocks each, 170 drawn
                                   (5, 256, 128256)])   # the 8B vocab: 7 blocks each, 212 drawn
def test_lm_head_fused_select_matches_reduce_launch(cuda, B, K, V):
    """The MFMA path's in-kernel selection (packed keys + ticket, with a
    counters buffer; from 1.5 blocks per workgroup on, blocks also drawn from
    a pool) gives the ids and logits of its partials + reduce-launch form
    (contiguous ranges), call after call, and leaves the counters at zero. Rows of zeros
    (every logit +-0: the smallest index wins), copied winners (ties) and a
    NaN row are included."""
    from llm_cuda import _native

    lib = _native.load()
    g = torch.Generator().manual_seed(B + K + V)
    hidden = torch.randn(B, K, generator=g).bfloat16()
    weight = (torch.randn(V, K, generator=g) * 0.02).bfloat16()
    hidden[0] = 0.0
    if V > 100:
        weight[V // 2] = weight[V // 3]
        weight[V - 1] = weight[7]
    if B > 2:
        hidden[1] = -hidden[2]
    hidden, weight = hidden.to(cuda), weight.to(cuda)
    n = lib.lc_lm_head_argmax_counter_count()
    counters = torch.zeros(n, dtype=torch.int32, device=cuda)
    ref_ids, ref_mx = _abi_call(hidden, weight, None)
    for call in range(3):
        ids, mx = _abi_call(hidden, weight, counters)
        torch.cuda.synchronize()
        assert torch.equal(ids, ref_ids), f"call {call}: ids differ"
        assert torch.equal(mx, ref_mx), f"call {call}: winning logits differ"
        assert not counters.any(), f"call {call}: counters not returned to zero"
    assert int(ref_ids[0]) == 0
    if V > 100:
        nan_w = weight.clone()
        nan_w[V // 4, 3] = float("nan")
        ids_n, _ = _abi_call(hidden, nan_w, counters)
        assert (ids_n.cpu() == V // 4).all()
        assert not counters.any()
