"""GPU parity: RMSNorm, SwiGLU, RoPE HIP kernels vs the fp32 oracle.

Shapes follow the reference's tests (test_cuda_extension.py, test_triton_swiglu.py,
test_triton_rope.py, seeds 40/21/99) plus the widths the reference's Triton
kernels got wrong (hidden/FFN > 4096) and strided / unaligned views that take
the element-wise path.
"""
import pytest
import torch

from helpers import ATOL, RTOL, assert_close
from oracle.elementwise import apply_rope, build_rope_cache, rms_norm, swiglu

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 4, 16), (3, 5, 256), (32, 1, 4096), (2, 3, 14336), (7, 100)])
def test_rmsnorm(cuda, dtype, shape):
    from llm_cuda.kernels.triton.rmsnorm import triton_rms_norm

    torch.manual_seed(40)
    x = torch.randn(*shape, device=cuda).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], device=cuda)).to(dtype)
    out = triton_rms_norm(x, w, 1e-5)
    assert out.dtype == dtype and out.shape == x.shape
    assert_close(out, rms_norm(x.cpu(), w.cpu(), 1e-5), ATOL[dtype], "rmsnorm", rtol=RTOL[dtype])


def test_rmsnorm_strided_rows_and_fp32_weight(cuda):
    from llm_cuda.kernels._ops import rms_norm as hip_rms

    torch.manual_seed(41)
    base = torch.randn(6, 300, device=cuda).to(torch.bfloat16)
    x = base[:, 10:266]  # row stride 300, unaligned start
    w = torch.randn(256, device=cuda)
    out = hip_rms(x, w, 1e-6)
    assert_close(out, rms_norm(x.cpu(), w.cpu(), 1e-6), ATOL[torch.bfloat16], "rmsnorm strided")


def test_rmsnorm_constant_row_closed_form(cuda):
    from llm_cuda.kernels.triton.rmsnorm import triton_rms_norm

    x = torch.full((4, 4096), 3.0, device=cuda)
    w = torch.linspace(0.5, 2.0, 4096, device=cuda)
    out = triton_rms_norm(x, w, 1e-5)
    assert_close(out, (3.0 * w / (9.0 + 1e-5) ** 0.5).expand(4, 4096), 1e-5, "const row")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 4, 16), (32, 1, 4096), (2, 20480), (3, 1001)])
@pytest.mark.parametrize("inplace", [False, True])
def test_add_rmsnorm(cuda, dtype, shape, inplace):
    """Fused residual add + RMSNorm: the sum equals torch's add in the storage
    dtype bit for bit, and y equals the oracle's rms_norm of that sum. Widths
    cover the register-cached path, the two-pass path (20480 > 256 lanes x 8
    vectors x 8) and the element-wise path (1001)."""
    from llm_cuda.kernels._ops import add_rms_norm

    torch.manual_seed(42)
    x = torch.randn(*shape, device=cuda).to(dtype)
    r = torch.randn(*shape, device=cuda).to(dtype)
    w = (1 + 0.1 * torch.randn(shape[-1], device=cuda)).to(dtype)
    ref_sum = x + r
    x_in = x.clone()
    y, s = add_rms_norm(x_in, r, w, 1e-5, inplace=inplace)
    assert torch.equal(s, ref_sum)
    if inplace:
        assert s.data_ptr() == x_in.data_ptr() and torch.equal(x_in, ref_sum)
    else:
        assert torch.equal(x_in, x)
    assert_close(y, rms_norm(ref_sum.cpu(), w.cpu(), 1e-5), ATOL[dtype], "add_rmsnorm",
                 rtol=RTOL[dtype])


def test_add_rmsnorm_strided_and_fp32_weight(cuda):
    from llm_cuda.kernels._ops import add_rms_norm

    torch.manual_seed(43)
    base = torch.randn(5, 600, device=cuda).to(torch.bfloat16)
    x, r = base[:, :256], base[:, 300:556]  # row stride 600
    w = torch.randn(256, device=cuda)
    y, s = add_rms_norm(x, r, w, 1e-6)
    assert torch.equal(s, x + r)
    assert_close(y, rms_norm((x + r).cpu(), w.cpu(), 1e-6), ATOL[torch.bfloat16], "strided")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 4, 16), (1, 8, 64), (32, 1, 14336), (3, 1001)])
def test_swiglu(cuda, dtype, shape):
    from llm_cuda.kernels.triton.swiglu import triton_swiglu

    torch.manual_seed(21)
    g = (torch.randn(*shape, device=cuda) * 3).to(dtype)
    u = torch.randn(*shape, device=cuda).to(dtype)
    out = triton_swiglu(g, u)
    assert out.dtype == dtype and out.shape == g.shape
    ref = swiglu(g.cpu(), u.cpu())
    assert_close(out, ref, ATOL[dtype], "swiglu", rtol=RTOL[dtype])


def test_swiglu_strided_rows(cuda):
    from llm_cuda.kernels._ops import swiglu as hip_swiglu

    torch.manual_seed(22)
    gu = torch.randn(5, 2 * 688, device=cuda, dtype=torch.bfloat16)
    g, u = gu[:, :688], gu[:, 688:]
    out = hip_swiglu(g, u)
    assert_close(out, swiglu(g.cpu(), u.cpu()), ATOL[torch.bfloat16], "swiglu strided")


def test_swiglu_special_values(cuda):
    from llm_cuda.kernels.triton.swiglu import triton_swiglu

    g = torch.tensor([0.0, 30.0, -30.0, -100.0, 100.0], device=cuda)
    u = torch.tensor([5.0, 2.0, 7.0, 1.0, 1.0], device=cuda)
    out = triton_swiglu(g, u).cpu()
    assert out[0] == 0 and abs(out[1] - 60) < 1e-4 and abs(out[2]) < 1e-9
    assert out[3] == 0 and abs(out[4] - 100) < 1e-4


def _proj_views(B, S, H, D, dtype, device, gen):
    """[B, H, S, D] views with the transposed-projection strides of _shape()."""
    x = torch.randn(B, S, H * D, generator=gen).to(dtype).to(device)
    return x.view(B, S, H, D).transpose(1, 2)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,H,S,D", [(2, 4, 16, 32), (1, 8, 32, 64), (1, 16, 1, 64), (4, 16, 64, 64),
                                     (1, 8, 16, 128)])
def test_rope_random_tables(cuda, dtype, B, H, S, D):
    """Random full-width tables (the reference's GPU test setup, test_triton_rope.py:110-122)."""
    from llm_cuda.kernels.triton.rope import can_use_triton_rope, triton_apply_rope

    gen = torch.Generator().manual_seed(99)
    x = torch.randn(B, H, S, D, generator=gen).to(dtype).to(cuda)
    cos = torch.randn(S, D, generator=gen).to(dtype).to(cuda)
    sin = torch.randn(S, D, generator=gen).to(dtype).to(cuda)
    assert can_use_triton_rope(x, cos, sin)
    out = triton_apply_rope(x, cos, sin)
    assert out.dtype == dtype and out.shape == x.shape and out.is_contiguous()
    ref = apply_rope(x.cpu(), cos.cpu(), sin.cpu())
    assert_close(out, ref, ATOL[dtype], "rope", rtol=RTOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rope_qk_strided_projection_views(cuda, dtype):
    """Q and K in one launch from the transposed projection views (no copies),
    with built tables at theta 500000 and a position offset."""
    from llm_cuda.models.llama3.rotary import apply_rotary

    gen = torch.Generator().manual_seed(98)
    B, S, Hq, Hkv, D = 2, 33, 8, 2, 128
    q = _proj_views(B, S, Hq, D, dtype, cuda, gen)
    k = _proj_views(B, S, Hkv, D, dtype, cuda, gen)
    cos, sin = build_rope_cache(S, D, 500000.0, dtype, position_offset=17)
    qo, ko = apply_rotary(q, k, cos.to(cuda), sin.to(cuda))
    assert_close(qo, apply_rope(q.cpu(), cos, sin), ATOL[dtype], "rope q")
    assert_close(ko, apply_rope(k.cpu(), cos, sin), ATOL[dtype], "rope k")


def test_rope_odd_half_scalar_path(cuda):
    from llm_cuda.kernels.triton.rope import triton_apply_rope

    gen = torch.Generator().manual_seed(97)
    x = torch.randn(2, 3, 5, 10, generator=gen).to(cuda)  # half = 5: element-wise path
    cos = torch.randn(5, 10, generator=gen).to(cuda)
    sin = torch.randn(5, 10, generator=gen).to(cuda)
    assert_close(triton_apply_rope(x, cos, sin), apply_rope(x.cpu(), cos.cpu(), sin.cpu()),
                 1e-5, "rope odd")


def test_predicates_true_on_device(cuda):
    from llm_cuda.kernels.triton.attention import can_use_triton_fused_attention
    from llm_cuda.kernels.triton.decode_attention import can_use_triton_decode_attention
    from llm_cuda.kernels.triton.rope import can_use_triton_rope

    q = torch.randn(1, 8, 1, 32, dtype=torch.float16, device=cuda)
    k = torch.randn(1, 4, 16, 32, dtype=torch.float16, device=cuda)
    assert can_use_triton_decode_attention(q, k, k) is True
    assert can_use_triton_decode_attention(q, k, k, attention_mask=k) is False
    assert can_use_triton_fused_attention(k, k, k) is True
    x = torch.randn(1, 8, 4, 64, device=cuda, dtype=torch.float16)
    c = torch.randn(4, 64, device=cuda, dtype=torch.float16)
    assert can_use_triton_rope(x, c, c) is True
    assert can_use_triton_rope(x[..., :63], c[:, :63], c[:, :63]) is False


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,hidden", [(32, 4096), (7, 1004), (3, 32768), (5, 14336)])
@pytest.mark.parametrize("n_parts", [1, 3, 4, 6])
def test_add_rmsnorm_over_partial_sums(cuda, dtype, rows, hidden, n_parts):
    """lc_add_rmsnorm_partials_fwd: the residual given as fp32 partials equals
    lc_add_rmsnorm_fwd with residual = round(0.0 + p_0 + p_1 + ...) bit for bit
    (y and the sum), over the row kernel's paths: vectors held in registers
    (4096, 14336), unaligned rows (1004), the two-pass loop (32768), and more
    than four partials (a second batch of loads)."""
    from llm_cuda.kernels import _ops

    g = torch.Generator(device=cuda).manual_seed(rows * 31 + hidden + n_parts)
    x = torch.randn(rows, 1, hidden, generator=g, device=cuda).to(dtype)
    parts = torch.randn(n_parts, rows, hidden, generator=g, device=cuda) * 0.5
    w = (1.0 + 0.1 * torch.randn(hidden, generator=g, device=cuda)).to(dtype)
    ps = _ops.PartialSum(parts, (rows, 1, hidden), dtype)
    r = ps.materialize()
    y, s = _ops.add_rms_norm(x, ps, w, 1e-5)
    y_ref, s_ref = _ops.add_rms_norm(x, r, w, 1e-5)
    assert torch.equal(s, s_ref) and torch.equal(y, y_ref)
    # in place, and with an fp32 weight
    x2 = x.clone()
    y2, s2 = _ops.add_rms_norm(x2, ps, w.float(), 1e-5, inplace=True)
    y2_ref, _ = _ops.add_rms_norm(x, r, w.float(), 1e-5)
    assert s2.data_ptr() == x2.data_ptr() and torch.equal(x2, s_ref) and torch.equal(y2, y2_ref)


def test_partial_sum_materialize_order(cuda):
    """PartialSum's value: fp32 partials added to 0.0 in order, then rounded
    (checked on values whose sum depends on the order)."""
    from llm_cuda.kernels import _ops

    big, tiny = 2.0 ** 24, 1.0
    parts = torch.tensor([[[big]], [[tiny]], [[-big]]], device=cuda)
    ps = _ops.PartialSum(parts, (1, 1), torch.float32)
    assert ps.materialize().item() == 0.0  # (big + 1) rounds to big in fp32, then - big
    rev = _ops.PartialSum(parts.flip(0), (1, 1), torch.float32)
    assert rev.materialize().item() == 1.0  # -big + 1 is exact, then + big
    mid = _ops.PartialSum(parts[[0, 2, 1]], (1, 1), torch.float32)
    assert mid.materialize().item() == 1.0


def test_add_rmsnorm_partials_layout_checked(cuda):
    """Partials that are not [S, rows, hidden] fp32 with unit stride over
    hidden are rejected before any launch."""
    from llm_cuda.kernels import _ops

    x = torch.randn(4, 256, device=cuda).bfloat16()
    w = torch.ones(256, device=cuda).bfloat16()
    good = torch.randn(2, 4, 256, device=cuda)
    bad = [torch.randn(2, 256, 4, device=cuda).transpose(1, 2),  # strided over hidden
           good.to(torch.float16),                                  # not fp32
           torch.randn(2, 4, 128, device=cuda)]                     # wrong width
    for parts in bad:
        with pytest.raises((ValueError, TypeError)):
            _ops.add_rms_norm(x, _ops.PartialSum(parts, (4, 256), x.dtype), w, 1e-5)
    _ops.add_rms_norm(x, _ops.PartialSum(good, (4, 256), x.dtype), w, 1e-5)
