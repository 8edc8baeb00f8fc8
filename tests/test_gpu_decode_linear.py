"""GPU parity: decode-step projections (lc_decode_linear) vs the oracle.

The oracle is the projection accumulated in fp64 and rounded once to the data
type (oracle/lm_head.py lm_head_logits, the nn.Linear output of the reference
at these shapes), and for mode 1 the reference's SwiGLU over the two rounded
projections (oracle/elementwise.py swiglu, rounded to the data type). The GPU
sums in fp32 in its own order (MFMA k-steps, then K-splits in split order),
so a value on a rounding boundary may land one ulp of the data type away:
the bar is one ulp of the result (relative), plus a floor of one ulp of the
output scale for values near zero. Mode 1 inherits one ulp on g and u, which
the SwiGLU at most doubles.
"""
import pytest
import torch

from oracle.elementwise import swiglu as oracle_swiglu
from oracle.lm_head import lm_head_logits

pytestmark = pytest.mark.gpu

ULP = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def _ref(x, w, swiglu):
    x2 = x.reshape(-1, x.shape[-1])
    if not swiglu:
        return lm_head_logits(x2, w).reshape(*x.shape[:-1], w.shape[0])
    n = w.shape[0] // 2
    g = lm_head_logits(x2, w[:n])
    u = lm_head_logits(x2, w[n:])
    return oracle_swiglu(g, u).to(x.dtype).reshape(*x.shape[:-1], n)


def _check(y, ref, ulps):
    y = y.detach().cpu().double()
    r = ref.double()
    scale = float(r.abs().max()) if r.numel() else 1.0
    tol = ulps * ULP[ref.dtype] * (r.abs() + scale * 2.0 ** -6)
    bad = ((y - r).abs() > tol)
    assert not bad.any(), (f"{int(bad.sum())} of {r.numel()} values off; max |d| "
                           f"{float((y - r).abs().max()):.3e} (scale {scale:.3e})")


def _inputs(M, N, K, dtype, swiglu, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(M, K, generator=g, device="cuda").to(dtype)
    rows = 2 * N if swiglu else N
    w = (torch.randn(rows, K, generator=g, device="cuda") * K ** -0.5).to(dtype)
    return x, w


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (5, 200, 512), (32, 4096, 4096),
                                   (17, 6144, 1024), (32, 384, 14336), (3, 1000, 256)])
@pytest.mark.parametrize("splits", [0, 1, 3, 8])
def test_plain_matches_oracle(dtype, M, N, K, splits):
    from llm_cuda.kernels import _ops

    x, w = _inputs(M, N, K, dtype, False, seed=M + N + K)
    y = _ops.decode_linear(x, w, splits=splits)
    assert y.shape == (M, N) and y.dtype == dtype
    _check(y, _ref(x, w, False), 1.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (7, 100, 512), (32, 14336, 4096),
                                   (32, 320, 2048)])
@pytest.mark.parametrize("splits", [0, 1, 4])
def test_swiglu_matches_oracle(dtype, M, N, K, splits):
    from llm_cuda.kernels import _ops

    x, w = _inputs(M, N, K, dtype, True, seed=M + N + K + 1)
    y = _ops.decode_linear(x, w, swiglu=True, splits=splits)
    assert y.shape == (M, N) and y.dtype == dtype
    _check(y, _ref(x, w, True), 3.0)


@pytest.mark.parametrize("swiglu,M,N,K,splits", [
    # 64-row blocks (K % 256 == 0), runs of 1-2 tiles that start and end
    # inside blocks
    (False, 32, 1000, 1280, 3),
    # 128-row blocks (K % 256 == 128), runs of 1-2 tiles
    (False, 9, 1000, 1152, 5),
    # mode 1 with 64-row blocks: runs of 4-5 tiles over 9-tile blocks
    (True, 32, 200, 2304, 2),
    # mode 1 with 128-row blocks
    (True, 7, 100, 384, 2),
    # a workgroup per tile: every block summed from all its tiles' partials
    (False, 4, 300, 3328, 13),
    # the library's grid on 256 CUs: 313 blocks of 5 tiles in runs of 7, so
    # a run can hold a whole block between two partial ones
    (False, 16, 20000, 1280, 0),
])
def test_runs_across_row_blocks(swiglu, M, N, K, splits):
    """Workgroup runs (equal shares of the (row block, K tile) units) that
    start and end inside row blocks, so blocks are summed from the partials of
    several workgroups, in both tile shapes and both modes."""
    from llm_cuda.kernels import _ops

    x, w = _inputs(M, N, K, torch.bfloat16, swiglu, seed=M * 7 + N + K)
    y = _ops.decode_linear(x, w, swiglu=swiglu, splits=splits)
    _check(y, _ref(x, w, swiglu), 3.0 if swiglu else 1.0)
    assert torch.equal(y, _ops.decode_linear(x, w, swiglu=swiglu, splits=splits))


def test_leading_dims_and_strided_rows():
    """x [B, 1, K] (the decode step's hidden states) and x rows with a stride
    past K (a column slice of a wider tensor)."""
    from llm_cuda.kernels import _ops

    x, w = _inputs(32, 768, 1024, torch.bfloat16, False, seed=5)
    y = _ops.decode_linear(x.view(32, 1, 1024), w)
    assert y.shape == (32, 1, 768)
    _check(y, _ref(x, w, False).view(32, 1, 768), 1.0)
    wide = torch.randn(9, 1024 + 256, device="cuda").bfloat16()
    xs = wide[:, 128:128 + 1024]
    y2 = _ops.decode_linear(xs, w, splits=2)
    _check(y2, _ref(xs, w, False), 1.0)


def test_consecutive_calls_reuse_workspace_and_counters():
    """Split partials and ticket counters are reused call after call: a second
    call with other inputs (and a smaller M) must not see the first's partials,
    and the counters must be back at zero after each call."""
    from llm_cuda.kernels import _ops

    w = (torch.randn(4096, 4096, device="cuda") * 4096 ** -0.5).bfloat16()
    for M, seed in ((32, 1), (32, 2), (9, 3), (1, 4)):
        g = torch.Generator(device="cuda").manual_seed(seed)
        x = torch.randn(M, 4096, generator=g, device="cuda").bfloat16()
        y = _ops.decode_linear(x, w, splits=8)
        _check(y, _ref(x, w, False), 1.0)
    torch.cuda.synchronize()
    dev = torch.device("cuda", torch.cuda.current_device())
    counters = _ops._COUNTERS[("decode_linear", "cuda", dev.index, _ops._stream(dev))]
    assert int(counters.abs().sum()) == 0


def test_counters_are_per_stream_and_odd_widths_route_elsewhere():
    """Calls on two streams (which may overlap) get separate ticket counters;
    an output width that is not a multiple of 4 is not taken (the library
    stores y rows 8 bytes at a time), so callers fall back to F.linear."""
    from llm_cuda.kernels import _ops

    x, w = _inputs(4, 512, 512, torch.bfloat16, False, seed=21)
    side = torch.cuda.Stream()
    y0 = _ops.decode_linear(x, w)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        y1 = _ops.decode_linear(x, w)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)
    dev = torch.device("cuda", torch.cuda.current_device())
    main = _ops._COUNTERS[("decode_linear", "cuda", dev.index, _ops._stream(dev))]
    other = _ops._COUNTERS[("decode_linear", "cuda", dev.index, side.cuda_stream)]
    assert main.data_ptr() != other.data_ptr()
    assert _ops.decode_linear_applies(x, w)
    assert not _ops.decode_linear_applies(x, w[:510])  # N = 510
    xo, wo = _inputs(4, 1001, 512, torch.bfloat16, False, seed=22)
    assert not _ops.decode_linear_applies(xo, wo)
    xs, ws = _inputs(4, 1001, 512, torch.bfloat16, True, seed=23)
    assert not _ops.decode_linear_applies(xs, ws, swiglu=True)


def test_deterministic_per_split_count():
    from llm_cuda.kernels import _ops

    x, w = _inputs(32, 4096, 4096, torch.bfloat16, False, seed=11)
    for splits in (0, 8, 16):
        a = _ops.decode_linear(x, w, splits=splits)
        b = _ops.decode_linear(x, w, splits=splits)
        assert torch.equal(a, b)


def test_graph_replay_matches_eager():
    """The ticket counters return to zero inside the kernel, so the launch can
    be captured and replayed; every replay is checked against eager."""
    from llm_cuda.kernels import _ops

    x, w = _inputs(32, 14336, 4096, torch.bfloat16, True, seed=21)
    eager = _ops.decode_linear(x, w, swiglu=True)
    x2, w2 = _inputs(32, 4096, 4096, torch.bfloat16, False, seed=22)
    eager2 = _ops.decode_linear(x2, w2, splits=8)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _ops.decode_linear(x, w, swiglu=True)
        _ops.decode_linear(x2, w2, splits=8)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = _ops.decode_linear(x, w, swiglu=True)
        y2 = _ops.decode_linear(x2, w2, splits=8)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
        assert torch.equal(y2, eager2)
        _ops.decode_linear(x2, w2, splits=8)  # eager work between replays
        torch.cuda.synchronize()


def test_c_abi_strided_output_and_errors():
    """y with a row stride past N through the C-ABI; argument errors."""
    from llm_cuda import _native as nat
    from llm_cuda.kernels import _ops

    lib = nat.load()
    x, w = _inputs(4, 256, 512, torch.bfloat16, False, seed=31)
    ybuf = torch.full((4, 300), 7.0, device="cuda").bfloat16()
    ws_bytes = lib.lc_decode_linear_workspace_bytes(4, 256, 512, 0, 2)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    counters = _ops._decode_linear_counters(x.device, 16)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.lc_decode_linear(x.data_ptr(), 512, w.data_ptr(), 512, ybuf.data_ptr(), 300, 4, 256,
                              512, 0, 2, ws.data_ptr(), ws.numel(), counters.data_ptr(),
                              nat.lc_dtype(x), stream)
    assert rc == 0
    torch.cuda.synchronize()
    _check(ybuf[:, :256], _ref(x, w, False), 1.0)
    assert bool((ybuf[:, 256:] == 7.0).all())
    bad = [
        (33, 256, 512, 0),   # M > 32
        (4, 256, 500, 0),    # K % 128
        (4, 256, 512, 2),    # unknown mode
    ]
    for M, N, K, mode in bad:
        rc = lib.lc_decode_linear(x.data_ptr(), 512, w.data_ptr(), 512, ybuf.data_ptr(), 300, M,
                                  N, K, mode, 0, ws.data_ptr(), ws.numel(), counters.data_ptr(),
                                  nat.lc_dtype(x), stream)
        assert rc != 0, (M, N, K, mode)
    # workspace too small for the split count
    rc = lib.lc_decode_linear(x.data_ptr(), 512, w.data_ptr(), 512, ybuf.data_ptr(), 300, 4, 256,
                              512, 0, 4, ws.data_ptr(), 16, counters.data_ptr(), nat.lc_dtype(x),
                              stream)
    assert rc != 0
    assert b"workspace" in lib.lc_last_error()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,shares", [
    (32, 4096, 4096, 0), (32, 4096, 14336, 0), (32, 4096, 4096, 4), (9, 1000, 1280, 5),
    (5, 256, 1152, 3), (1, 64, 128, 1), (32, 6144, 4096, 2), (3, 300, 2304, 9)])
def test_partials_sum_equals_decode_linear(dtype, M, N, K, shares):
    """lc_decode_linear_partials: the shares' fp32 partials, added to 0.0 in
    share order and rounded, equal lc_decode_linear's output bit for bit at
    the same share count (the same tiles per share and the same sum order), and
    the oracle to one ulp. Covers both tile shapes (K % 256 == 0 and == 128)
    and the library's share choice."""
    from llm_cuda import _native as nat
    from llm_cuda.kernels import _ops

    x, w = _inputs(M, N, K, dtype, False, seed=M + 3 * N + K)
    ps = _ops.decode_linear_partials(x, w, shares=shares)
    S = ps.parts.shape[0]
    if shares == 0:
        assert S == nat.load().lc_decode_linear_partial_count(N, K)
    assert ps.parts.shape == (S, M, N) and ps.shape == (M, N) and ps.dtype == dtype
    y = ps.materialize()
    assert torch.equal(y, _ops.decode_linear(x, w, splits=S))
    _check(y, _ref(x, w, False), 1.0)


def test_partials_arguments_rejected():
    """Shares that do not divide a row block's tiles, N % 4 != 0, misaligned
    partials: errors before any launch."""
    from llm_cuda import _native as nat

    lib = nat.load()
    x, w = _inputs(4, 256, 1024, torch.bfloat16, False, seed=41)  # 64-row blocks of 4 tiles
    parts = torch.empty(8, 4, 256, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for N, shares, off, what in ((256, 3, 0, b"divide"), (254, 1, 0, b"N=254"),
                                 (256, 2, 4, b"aligned")):
        rc = lib.lc_decode_linear_partials(x.data_ptr(), 1024, w.data_ptr(), 1024,
                                           parts.data_ptr() + off, 4, N, 1024, shares,
                                           nat.lc_dtype(x), stream)
        assert rc != 0 and what in lib.lc_last_error(), lib.lc_last_error()
    assert lib.lc_decode_linear_partial_count(256, 1000) == -1
