"""Tensor-level wrappers over the C ABI (include/lcuda.h).

Every function here validates shapes on the host, allocates outputs and
workspace through torch's caching allocator on the inputs' device, and
launches on torch's current stream of that device. Inputs must be ROCm
device tensors; anything else raises (there is no second implementation).
"""
from __future__ import annotations

import contextlib
import math

import torch

from llm_cuda import _native as nat


def _i64arr(vals):
    import ctypes

    return (ctypes.c_int64 * len(vals))(*vals)


def _stream(dev: torch.device) -> int:
    return nat.stream_ptr(dev)


_CU_COUNTS: dict[int, int] = {}


def _cu_count(dev: torch.device) -> int:
    """Compute units of the device (cached per device index)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    n = _CU_COUNTS.get(idx)
    if n is None:
        n = _CU_COUNTS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return n


class _DeviceGuard:
    """Make `dev` current for the launch if it is not already."""

    def __init__(self, dev: torch.device):
        self.dev = dev
        self.prev = None

    def __enter__(self):
        idx = self.dev.index if self.dev.index is not None else torch.cuda.current_device()
        cur = torch.cuda.current_device()
        if cur != idx:
            self.prev = cur
            torch.cuda.set_device(idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


# ---------------------------------------------------------------------------
# Forward-only kernels under autograd
# ---------------------------------------------------------------------------
class _ForwardOnly(torch.autograd.Function):
    """Runs a forward-only kernel inside the autograd graph so that a backward
    pass through its outputs raises instead of silently skipping every input
    upstream of it (the kernel has no backward in this build)."""

    @staticmethod
    def forward(ctx, name, fn, *inputs):
        ctx.name = name
        return fn(*inputs)

    @staticmethod
    def backward(ctx, *grads):
        raise NotImplementedError(
            f"{ctx.name} has no backward in this build (inference path only); run the "
            "forward under torch.no_grad() or with inputs that do not require grad")


def _records_grad(*tensors) -> bool:
    return torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in tensors)


# ---------------------------------------------------------------------------
# RMSNorm  (reference: kernels/triton/rmsnorm.py:46-75, norm.py:22-33)
# ---------------------------------------------------------------------------
def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * weight over the last dimension (forward only)."""
    if _records_grad(x, weight):
        return _ForwardOnly.apply("rms_norm", lambda a, w: _rms_norm(a, w, eps), x, weight)
    return _rms_norm(x, weight, eps)


def _rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    dev = nat.require_device(x, weight)
    if weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(f"weight shape {tuple(weight.shape)} does not match hidden {x.shape[-1]}")
    hidden = x.shape[-1]
    x2 = x.reshape(-1, hidden)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w = weight if weight.is_contiguous() else weight.contiguous()
    if w.dtype != x.dtype and w.dtype != torch.float32:
        w = w.to(x.dtype)
    y = torch.empty((x2.shape[0], hidden), dtype=x.dtype, device=dev)
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_rmsnorm_fwd(
            x2.data_ptr(), w.data_ptr(), y.data_ptr(), x2.shape[0], hidden, x2.stride(0),
            y.stride(0), float(eps), nat.lc_dtype(x), nat.lc_dtype(w), _stream(dev))
    nat.check(rc, "lc_rmsnorm_fwd")
    return y.view(x.shape)


def add_rms_norm(x: torch.Tensor, residual, weight: torch.Tensor, eps: float,
                 inplace: bool = False):
    """s = x + residual (rounded to x's dtype), y = rms_norm(s) * weight; returns (y, s).

    One pass over the rows instead of an add and a norm (reference pair:
    models/llama3/model.py:29-42). With inplace=True, s is written into x.
    residual may be a PartialSum (a projection's split-K partials, see
    decode_linear_partials): its sum is formed in the same pass.
    Forward only: a backward through y or s raises.
    """
    if isinstance(residual, PartialSum):
        if _records_grad(x, weight):
            raise NotImplementedError("add_rms_norm over partial sums is forward-only")
        return _add_rms_norm_partials(x, residual, weight, eps, inplace)
    if _records_grad(x, residual, weight):
        if inplace:
            raise NotImplementedError(
                "in-place add_rms_norm cannot be recorded by autograd (forward-only kernel)")
        return _ForwardOnly.apply(
            "add_rms_norm", lambda a, r, w: _add_rms_norm(a, r, w, eps, False), x, residual,
            weight)
    return _add_rms_norm(x, residual, weight, eps, inplace)


def _add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
                  inplace: bool):
    dev = nat.require_device(x, residual, weight)
    if x.shape != residual.shape or x.dtype != residual.dtype:
        raise ValueError("x and residual must have the same shape and dtype")
    if weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(f"weight shape {tuple(weight.shape)} does not match hidden {x.shape[-1]}")
    hidden = x.shape[-1]
    x2 = x.reshape(-1, hidden)
    r2 = residual.reshape(-1, hidden)
    if inplace and (x2.data_ptr() != x.data_ptr() or x2.stride(-1) != 1):
        raise ValueError("inplace add_rms_norm needs x with unit stride over hidden")
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if r2.stride(-1) != 1:
        r2 = r2.contiguous()
    w = weight if weight.is_contiguous() else weight.contiguous()
    if w.dtype != x.dtype and w.dtype != torch.float32:
        w = w.to(x.dtype)
    y = torch.empty((x2.shape[0], hidden), dtype=x.dtype, device=dev)
    s2 = x2 if inplace else torch.empty((x2.shape[0], hidden), dtype=x.dtype, device=dev)
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_add_rmsnorm_fwd(
            x2.data_ptr(), r2.data_ptr(), w.data_ptr(), y.data_ptr(), s2.data_ptr(), x2.shape[0],
            hidden, x2.stride(0), r2.stride(0), y.stride(0), s2.stride(0), float(eps),
            nat.lc_dtype(x), nat.lc_dtype(w), _stream(dev))
    nat.check(rc, "lc_add_rmsnorm_fwd")
    return y.view(x.shape), (x if inplace else s2.view(x.shape))


def _add_rms_norm_partials(x: torch.Tensor, residual: "PartialSum", weight: torch.Tensor,
                           eps: float, inplace: bool):
    dev = nat.require_device(x, residual.parts, weight)
    if tuple(residual.shape) != tuple(x.shape) or residual.dtype != x.dtype:
        raise ValueError(f"partial sum {tuple(residual.shape)} {residual.dtype} does not match "
                         f"x {tuple(x.shape)} {x.dtype}")
    if weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(f"weight shape {tuple(weight.shape)} does not match hidden {x.shape[-1]}")
    hidden = x.shape[-1]
    x2 = x.reshape(-1, hidden)
    if inplace and (x2.data_ptr() != x.data_ptr() or x2.stride(-1) != 1):
        raise ValueError("inplace add_rms_norm needs x with unit stride over hidden")
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w = weight if weight.is_contiguous() else weight.contiguous()
    if w.dtype != x.dtype and w.dtype != torch.float32:
        w = w.to(x.dtype)
    parts = residual.parts  # [S, rows, hidden] fp32, unit stride over hidden
    if (parts.dtype != torch.float32 or parts.dim() != 3
            or tuple(parts.shape[1:]) != (x2.shape[0], hidden) or parts.stride(2) != 1):
        raise ValueError(f"partials must be fp32 [S, {x2.shape[0]}, {hidden}] with unit stride "
                         f"over hidden; got {tuple(parts.shape)} strides {parts.stride()}")
    y = torch.empty((x2.shape[0], hidden), dtype=x.dtype, device=dev)
    s2 = x2 if inplace else torch.empty((x2.shape[0], hidden), dtype=x.dtype, device=dev)
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_add_rmsnorm_partials_fwd(
            x2.data_ptr(), parts.data_ptr(), parts.shape[0], parts.stride(0), w.data_ptr(),
            y.data_ptr(), s2.data_ptr(), x2.shape[0], hidden, x2.stride(0), parts.stride(1),
            y.stride(0), s2.stride(0), float(eps), nat.lc_dtype(x), nat.lc_dtype(w), _stream(dev))
    nat.check(rc, "lc_add_rmsnorm_partials_fwd")
    return y.view(x.shape), (x if inplace else s2.view(x.shape))


# ---------------------------------------------------------------------------
# SwiGLU  (reference: kernels/triton/swiglu.py:91-145,199-200)
# ---------------------------------------------------------------------------
def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up in fp32, rounded to gate's dtype (forward only)."""
    if _records_grad(gate, up):
        return _ForwardOnly.apply("swiglu", _swiglu, gate, up)
    return _swiglu(gate, up)


def _swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    if gate.shape != up.shape:
        raise ValueError("gate and up must have matching shapes")
    if gate.dtype != up.dtype:
        raise TypeError("gate and up must have the same dtype")
    dev = nat.require_device(gate, up)
    if gate.numel() == 0:
        return torch.empty(gate.shape, dtype=gate.dtype, device=dev)
    cols = gate.shape[-1] if gate.dim() > 0 else 1
    g2 = gate.reshape(-1, cols)
    u2 = up.reshape(-1, cols)
    if g2.stride(-1) != 1:
        g2 = g2.contiguous()
    if u2.stride(-1) != 1:
        u2 = u2.contiguous()
    out = torch.empty((g2.shape[0], cols), dtype=gate.dtype, device=dev)
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_swiglu_fwd(
            g2.data_ptr(), u2.data_ptr(), out.data_ptr(), g2.shape[0], cols, g2.stride(0),
            u2.stride(0), out.stride(0), nat.lc_dtype(gate), _stream(dev))
    nat.check(rc, "lc_swiglu_fwd")
    return out.view(gate.shape)


# ---------------------------------------------------------------------------
# RoPE  (reference: kernels/triton/rope.py:156-222, rotary.py:81-109)
# ---------------------------------------------------------------------------
def _check_rope_operand(x: torch.Tensor, cos: torch.Tensor, name: str) -> None:
    if x.dim() != 4:
        raise ValueError(f"{name} must be [batch, heads, seq, head_dim], got {tuple(x.shape)}")
    if x.shape[-1] % 2 != 0:
        raise ValueError(f"{name} head_dim must be even")
    if tuple(cos.shape) != (x.shape[-2], x.shape[-1]):
        raise ValueError(
            f"cos/sin shape {tuple(cos.shape)} must be [seq, head_dim] = "
            f"{(x.shape[-2], x.shape[-1])}")
    if x.dtype != cos.dtype:
        raise TypeError(f"{name} dtype {x.dtype} differs from cos/sin dtype {cos.dtype}")


def rope(x1: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
         x2: torch.Tensor | None = None):
    """Rotate x1 (and x2) in one launch; returns contiguous new tensors (forward only)."""
    if _records_grad(x1, x2, cos, sin):
        if x2 is None:
            return _ForwardOnly.apply("rope", lambda a, c, s_: _rope(a, c, s_, None)[0], x1,
                                      cos, sin), None
        return _ForwardOnly.apply("rope", _rope, x1, cos, sin, x2)
    return _rope(x1, cos, sin, x2)


def _rope(x1: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
          x2: torch.Tensor | None = None):
    if cos.shape != sin.shape or cos.dtype != sin.dtype:
        raise ValueError("cos and sin must have the same shape and dtype")
    _check_rope_operand(x1, cos, "x")
    if x2 is not None:
        _check_rope_operand(x2, cos, "k")
        if x2.shape[0] != x1.shape[0] or x2.shape[2:] != x1.shape[2:]:
            raise ValueError("q and k must share batch, seq and head_dim")
    dev = nat.require_device(x1, cos, sin, x2)
    if x1.stride(-1) != 1:
        x1 = x1.contiguous()
    if x2 is not None and x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if cos.stride(-1) != 1:
        cos = cos.contiguous()
    if sin.stride(-1) != 1:
        sin = sin.contiguous()
    B, H1, S, D = x1.shape
    o1 = torch.empty((B, H1, S, D), dtype=x1.dtype, device=dev)
    o2 = None if x2 is None else torch.empty(tuple(x2.shape), dtype=x2.dtype, device=dev)
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_rope_fwd(
            x1.data_ptr(), o1.data_ptr(), H1, _i64arr(x1.stride()), _i64arr(o1.stride()),
            None if x2 is None else x2.data_ptr(), None if o2 is None else o2.data_ptr(),
            0 if x2 is None else x2.shape[1],
            None if x2 is None else _i64arr(x2.stride()),
            None if o2 is None else _i64arr(o2.stride()),
            cos.data_ptr(), sin.data_ptr(), cos.stride(0), sin.stride(0), B, S, D,
            nat.lc_dtype(x1), _stream(dev))
    nat.check(rc, "lc_rope_fwd")
    return o1, o2


# ---------------------------------------------------------------------------
# Additive attention masks
# ---------------------------------------------------------------------------
def _mask_dtype(mask: torch.Tensor, data_dtype: torch.dtype) -> torch.Tensor:
    """An additive mask in a dtype the kernels read: fp32 or the data dtype
    (other floating dtypes are widened to fp32; non-float masks are refused,
    since the reference adds the mask to the scores)."""
    if not mask.is_floating_point():
        raise TypeError(f"attention_mask must be a floating-point additive mask, got {mask.dtype}")
    if mask.dtype not in (torch.float32, data_dtype):
        mask = mask.float()
    return mask


def prefill_bias(mask: torch.Tensor, B: int, Hq: int, Sq: int, Skv: int,
                 data_dtype: torch.dtype) -> torch.Tensor:
    """The additive mask as a [B, Hq, Sq, Skv] view (broadcast dimensions get
    stride 0; nothing is copied unless the dtype must change)."""
    mask = _mask_dtype(mask, data_dtype)
    try:
        return mask.expand(B, Hq, Sq, Skv)
    except RuntimeError as exc:
        raise ValueError(f"attention_mask of shape {tuple(mask.shape)} does not broadcast to "
                         f"[batch, heads, q_len, kv_len] = {(B, Hq, Sq, Skv)}") from exc


def decode_bias(mask: torch.Tensor, B: int, Hq: int, data_dtype: torch.dtype) -> torch.Tensor:
    """The additive mask of one query token as a [B, Hq, L] view with unit token
    stride (L = the mask's last dimension); accepts [.., 1, L] and [.., L] forms
    broadcastable to [B, Hq, 1, L]."""
    mask = _mask_dtype(mask, data_dtype)
    if mask.dim() == 4:
        if mask.shape[2] != 1:
            raise ValueError(f"a decode mask has one query row, got shape {tuple(mask.shape)}")
        mask = mask[:, :, 0]
    L = mask.shape[-1]
    try:
        m = mask.expand(B, Hq, L)
    except RuntimeError as exc:
        raise ValueError(f"attention_mask of shape {tuple(mask.shape)} does not broadcast to "
                         f"[batch, heads, kv_len] = {(B, Hq, L)}") from exc
    if L > 1 and m.stride(-1) != 1:
        m = m.contiguous()
    return m


# ---------------------------------------------------------------------------
# Prefill attention  (reference: kernels/triton/attention.py:323-378,501-535)
# ---------------------------------------------------------------------------
def prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_offset: int = 0,
                      scale: float | None = None, return_lse: bool = False,
                      attention_mask: torch.Tensor | None = None):
    """Causal attention of q [B, Hq, Sq, D] over k, v [B, Hkv, Skv, D]; key j is
    visible to query i iff j <= i + q_offset. attention_mask: an additive mask
    broadcastable to [B, Hq, Sq, Skv] (fp32 or q's dtype), added to the scaled
    scores as in the reference's torch path (attention.py:457-477)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [batch, heads, seq, head_dim]")
    if k.shape != v.shape:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} shapes differ")
    B, Hq, Sq, D = q.shape
    if k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} are incompatible")
    Hkv, Skv = k.shape[1], k.shape[2]
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"n_heads ({Hq}) must be a multiple of n_kv_heads ({Hkv})")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    dev = nat.require_device(q, k, v)
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    bias = None
    if attention_mask is not None:
        nat.require_device(q, attention_mask)
        bias = prefill_bias(attention_mask, B, Hq, Sq, Skv, q.dtype)
    out = torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=dev)
    lse = torch.empty((B, Hq, Sq), dtype=torch.float32, device=dev) if return_lse else None
    lib = nat.load()
    # The ticket of the kernel's dynamic tail (zero-on-exit); a capture before
    # any eager call runs the static order (no counters).
    counters = _zeroed_counters("prefill", dev, lib.lc_prefill_attn_counter_count(),
                                optional=True)
    with _DeviceGuard(dev):
        rc = lib.lc_prefill_attn_fwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            None if lse is None else lse.data_ptr(), B, Hq, Hkv, Sq, Skv, D,
            _i64arr(q.stride()), _i64arr(k.stride()), _i64arr(v.stride()), _i64arr(out.stride()),
            int(q_offset), None if bias is None else bias.data_ptr(),
            None if bias is None else _i64arr(bias.stride()),
            0 if bias is None else nat.lc_dtype(bias),
            None if counters is None else counters.data_ptr(), float(scale), nat.lc_dtype(q),
            _stream(dev))
    nat.check(rc, "lc_prefill_attn_fwd")
    return (out, lse) if return_lse else out


def prefill_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               out: torch.Tensor, lse: torch.Tensor, dout: torch.Tensor,
                               q_offset: int = 0, scale: float | None = None,
                               attention_mask: torch.Tensor | None = None):
    """(dq, dk, dv) of causal attention (reference: kernels/triton/attention.py:380-454).

    `out` and `lse` are the forward's output and fp32 natural-log logsumexp,
    computed with the same attention_mask (which gets no gradient). dk and dv
    are summed over the query heads that share a kv head.
    """
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [batch, heads, seq, head_dim]")
    if k.shape != v.shape:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} shapes differ")
    B, Hq, Sq, D = q.shape
    if k.shape[0] != B or k.shape[3] != D:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} are incompatible")
    Hkv, Skv = k.shape[1], k.shape[2]
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"n_heads ({Hq}) must be a multiple of n_kv_heads ({Hkv})")
    if out.shape != q.shape or dout.shape != q.shape:
        raise ValueError("out and dout must have q's shape")
    if lse.shape != (B, Hq, Sq) or lse.dtype != torch.float32:
        raise ValueError("lse must be fp32 [batch, heads, seq]")
    if not (q.dtype == k.dtype == v.dtype == out.dtype == dout.dtype):
        raise TypeError("q, k, v, out, dout must share a dtype")
    dev = nat.require_device(q, k, v, out, lse, dout)
    q, k, v, out, dout = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v, out, dout))
    lse = lse.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    bias = None
    if attention_mask is not None:
        nat.require_device(q, attention_mask)
        bias = prefill_bias(attention_mask, B, Hq, Sq, Skv, q.dtype)
    dq = torch.empty((B, Hq, Sq, D), dtype=q.dtype, device=dev)
    dk = torch.empty((B, Hkv, Skv, D), dtype=q.dtype, device=dev)
    dv = torch.empty((B, Hkv, Skv, D), dtype=q.dtype, device=dev)
    lib = nat.load()
    ws_bytes = lib.lc_prefill_attn_bwd_workspace_bytes(B, Hq, Sq)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    with _DeviceGuard(dev):
        rc = lib.lc_prefill_attn_bwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
            dout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, Hq, Hkv, Sq, Skv, D,
            _i64arr(q.stride()), _i64arr(k.stride()), _i64arr(v.stride()),
            _i64arr(out.stride()), _i64arr(dout.stride()), _i64arr(dq.stride()),
            _i64arr(dk.stride()), _i64arr(dv.stride()), int(q_offset),
            None if bias is None else bias.data_ptr(),
            None if bias is None else _i64arr(bias.stride()),
            0 if bias is None else nat.lc_dtype(bias), float(scale), ws.data_ptr(), ws.numel(),
            nat.lc_dtype(q), _stream(dev))
    nat.check(rc, "lc_prefill_attn_bwd")
    return dq, dk, dv


# ---------------------------------------------------------------------------
# lm_head + greedy argmax  (reference: models/llama3/model.py:156,214)
# ---------------------------------------------------------------------------
def lm_head_argmax(hidden: torch.Tensor, weight: torch.Tensor, return_max: bool = False):
    """ids[b] = argmax_v round(hidden[b] . weight[v]) for hidden [B, K], weight [V, K].

    The logits are rounded to hidden's dtype before the comparison (the
    reference takes argmax over lm_head's output in the model dtype); NaN
    ranks highest and ties go to the smallest index, as in torch.argmax.
    Returns int64 ids [B] (and the winning logits as fp32 [B] with return_max).
    """
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"hidden {tuple(hidden.shape)} and weight {tuple(weight.shape)} "
                         "must be [B, K] and [V, K]")
    if hidden.dtype != weight.dtype:
        raise TypeError("hidden and weight must share a dtype")
    dev = nat.require_device(hidden, weight)
    hidden = hidden if hidden.stride(-1) == 1 else hidden.contiguous()
    weight = weight if weight.stride(-1) == 1 else weight.contiguous()
    B, K = hidden.shape
    # The MFMA path addresses the hidden rows of one 32-row chunk with 32-bit
    # byte offsets (the library's own condition); a widely strided view (the
    # last position of a long prompt) is packed first (B x K elements) rather
    # than sent to the generic kernel.
    if B > 1 and ((min(B, 32) - 1) * hidden.stride(0) + K) * hidden.element_size() >= 2 ** 31:
        hidden = hidden.contiguous()
    V = weight.shape[0]
    ids = torch.empty(B, dtype=torch.int64, device=dev)
    mx = torch.empty(B, dtype=torch.float32, device=dev) if return_max else None
    lib = nat.load()
    ws_bytes = lib.lc_lm_head_argmax_workspace_bytes(B, V)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    counters = _zeroed_counters("lm_head", dev, lib.lc_lm_head_argmax_counter_count())
    with _DeviceGuard(dev):
        rc = lib.lc_lm_head_argmax(
            hidden.data_ptr(), hidden.stride(0), weight.data_ptr(), weight.stride(0), B, K, V,
            ids.data_ptr(), None if mx is None else mx.data_ptr(), ws.data_ptr(), ws.numel(),
            counters.data_ptr(), nat.lc_dtype(hidden), _stream(dev))
    nat.check(rc, "lc_lm_head_argmax")
    return (ids, mx) if return_max else ids


# ---------------------------------------------------------------------------
# Decode-step projections  (reference: the nn.Linear calls of
# models/llama3/attention.py:100-102,154 and mlp.py:35-43 at a decode step)
# ---------------------------------------------------------------------------
DECODE_LINEAR_MAX_ROWS = 32
_NATIVE_PROJECTIONS = [True]
_COUNTERS: dict = {}
# Counter buffers replaced by a larger one stay referenced here: a HIP graph
# captured earlier may still hold their addresses.
_RETIRED_COUNTERS: list = []


def _zeroed_counters(kind: str, dev: torch.device, n: int, optional: bool = False):
    """Zeroed int32 counters for the kernels that take them (`kind`:
    "decode_linear" ticket counters, "lm_head" argmax keys and ticket,
    "paged_decode" the ticket of the longest-first order's dynamic tail,
    "prefill" the ticket of the prefill kernel's dynamic tail). Each
    call leaves its counters at zero, so calls that follow one another on a
    stream can share a buffer; calls on different streams (which may overlap)
    must not. Eager calls get one buffer per (kind, device, stream). Calls
    captured into HIP graphs share one more buffer per (kind, device) (a
    capture cannot allocate and zero it: every eager call makes sure it
    exists), so replays of graphs holding such calls must not overlap on one
    device. A capture before any eager call raises, or returns None when
    `optional` (for kernels whose counters are an optimisation only)."""
    capturing = torch.cuda.is_current_stream_capturing()
    keys = [(kind, dev.type, dev.index, "graphs")]
    if not capturing:
        keys.append((kind, dev.type, dev.index, _stream(dev)))
    for key in keys:
        buf = _COUNTERS.get(key)
        if buf is None or buf.numel() < n:
            if capturing:
                if optional:
                    return None
                raise RuntimeError(f"{kind}: run one call outside graph capture first "
                                   "(its counters are allocated and zeroed eagerly)")
            if buf is not None:
                _RETIRED_COUNTERS.append(buf)
            buf = torch.zeros(max(n, 4096), dtype=torch.int32, device=dev)
            _COUNTERS[key] = buf
    return buf


def _decode_linear_counters(dev: torch.device, n: int) -> torch.Tensor:
    return _zeroed_counters("decode_linear", dev, n)


@contextlib.contextmanager
def torch_projections():
    """Within the block, the model's decode-step projections run as torch
    matmuls (F.linear, hipBLASLt on ROCm) instead of lc_decode_linear: every
    decode_linear_applies answers False. This is the reference's own
    projection path (nn.Linear, models/llama3/attention.py:100-102,154 and
    mlp.py:39-43); the attention, RoPE, KV append, RMSNorm and SwiGLU kernels
    are the same either way. Not thread-safe: it flips a module-wide switch."""
    prev = _NATIVE_PROJECTIONS[0]
    _NATIVE_PROJECTIONS[0] = False
    try:
        yield
    finally:
        _NATIVE_PROJECTIONS[0] = prev


def native_projections() -> bool:
    """False inside torch_projections(): the decode-step projections are torch
    matmuls there."""
    return _NATIVE_PROJECTIONS[0]


def decode_linear_applies(x: torch.Tensor, weight: torch.Tensor, swiglu: bool = False) -> bool:
    """True where decode_linear takes the call: bf16/f16 on the GPU, 1-32 rows,
    K % 128 == 0, an output width N % 4 == 0, aligned rows, no autograd graph
    being recorded, and not inside torch_projections()."""
    if not _NATIVE_PROJECTIONS[0]:
        return False
    if not (x.is_cuda and weight.is_cuda and x.dtype == weight.dtype
            and x.dtype in (torch.bfloat16, torch.float16) and weight.dim() == 2):
        return False
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    if not (1 <= rows <= DECODE_LINEAR_MAX_ROWS and K % 128 == 0 and weight.shape[1] == K):
        return False
    if swiglu and weight.shape[0] % 2:
        return False
    # lc_decode_linear writes y rows of N elements with 8-byte stores
    if (weight.shape[0] // 2 if swiglu else weight.shape[0]) % 4:
        return False
    if _records_grad(x, weight):
        return False
    return (weight.stride(1) == 1 and weight.stride(0) % 8 == 0
            and weight.data_ptr() % 16 == 0)


def decode_linear(x: torch.Tensor, weight: torch.Tensor, swiglu: bool = False,
                  splits: int = 0) -> torch.Tensor:
    """Projection of a decode step's rows, the weight streamed once.

    swiglu=False: x @ weight.T (weight [N, K], nn.Linear layout), rounded to
    x's dtype. swiglu=True: weight is [gate; up] ([2N, K]) and the result is
    swiglu(x @ gate.T, x @ up.T) with both projections rounded first (the
    reference's gate_proj / up_proj outputs). x: [..., K] with at most 32 rows.
    splits: workgroups per row block of the weight (0 = the library's choice:
    equal shares of the weight's tiles, one workgroup per CU).
    """
    if _records_grad(x, weight):
        raise RuntimeError("decode_linear is inference-only (autograd is recording)")
    if x.dtype != weight.dtype:
        raise TypeError("x and weight must share a dtype")
    if weight.dim() != 2 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"x {tuple(x.shape)} and weight {tuple(weight.shape)} do not match")
    dev = nat.require_device(x, weight)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    weight = weight if weight.stride(-1) == 1 else weight.contiguous()
    M = x2.shape[0]
    N = weight.shape[0] // 2 if swiglu else weight.shape[0]
    y = torch.empty(*lead, N, dtype=x.dtype, device=dev)
    if M == 0:
        return y
    mode = 1 if swiglu else 0
    lib = nat.load()
    ws_bytes = lib.lc_decode_linear_workspace_bytes(M, N, K, mode, int(splits))
    if ws_bytes < 0:
        raise ValueError(f"decode_linear: unsupported sizes M={M} N={N} K={K}")
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    counters = _decode_linear_counters(dev, lib.lc_decode_linear_counter_count(N, mode))
    with _DeviceGuard(dev):
        rc = lib.lc_decode_linear(
            x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0), y.data_ptr(), N,
            M, N, K, mode, int(splits), ws.data_ptr(), ws.numel(), counters.data_ptr(),
            nat.lc_dtype(x), _stream(dev))
    nat.check(rc, "lc_decode_linear")
    return y


class PartialSum:
    """A projection's output left as fp32 split-K partials: the value is
    round(0.0 + parts[0] + parts[1] + ...) in `dtype`, summed in that order
    (what decode_linear itself writes when its split is the same). parts: [S, rows, N] fp32; `shape` is
    the projection output's shape. add_rms_norm takes it as its residual and
    forms the sum in its own pass; materialize() forms it on its own."""

    def __init__(self, parts: torch.Tensor, shape, dtype: torch.dtype):
        self.parts = parts
        self.shape = torch.Size(shape)
        self.dtype = dtype

    @property
    def device(self) -> torch.device:
        return self.parts.device

    def materialize(self) -> torch.Tensor:
        acc = torch.zeros_like(self.parts[0])
        for p in self.parts:
            acc = acc + p
        return acc.to(self.dtype).view(self.shape)


def decode_linear_partials_applies(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """decode_linear_applies, plus N % 4 == 0 (the partials' float4 rows)."""
    return decode_linear_applies(x, weight) and weight.shape[0] % 4 == 0


def decode_linear_partials(x: torch.Tensor, weight: torch.Tensor, shares: int = 0) -> PartialSum:
    """x @ weight.T (weight [N, K]) with the split-K sum left undone: a
    PartialSum whose value equals decode_linear(x, weight) up to the order of
    the fp32 split-K sums. It is bit-identical where lc_decode_linear's default
    grid deals each row block out in equal whole K-shares (the library's
    default `shares` is then that same split); elsewhere the K split, and so
    the summation order, differs. shares: K-shares per row block of the
    weight (0 = the library's choice)."""
    if _records_grad(x, weight):
        raise RuntimeError("decode_linear_partials is inference-only (autograd is recording)")
    if x.dtype != weight.dtype:
        raise TypeError("x and weight must share a dtype")
    if weight.dim() != 2 or x.shape[-1] != weight.shape[1]:
        raise ValueError(f"x {tuple(x.shape)} and weight {tuple(weight.shape)} do not match")
    dev = nat.require_device(x, weight)
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    weight = weight if weight.stride(-1) == 1 else weight.contiguous()
    M, N = x2.shape[0], weight.shape[0]
    lib = nat.load()
    S = int(shares) if shares > 0 else lib.lc_decode_linear_partial_count(N, K)
    if S < 1:
        raise ValueError(f"decode_linear_partials: unsupported sizes N={N} K={K}")
    parts = torch.empty(S, M, N, dtype=torch.float32, device=dev)
    if M:
        with _DeviceGuard(dev):
            rc = lib.lc_decode_linear_partials(
                x2.data_ptr(), x2.stride(0), weight.data_ptr(), weight.stride(0),
                parts.data_ptr(), M, N, K, S, nat.lc_dtype(x), _stream(dev))
        nat.check(rc, "lc_decode_linear_partials")
    return PartialSum(parts, (*lead, N), x.dtype)


# ---------------------------------------------------------------------------
# Paged decode  (reference: kernels/triton/decode_attention.py:204-287 over
# models/llama3/kv_cache.py:65-83)
# ---------------------------------------------------------------------------
def _workgroup_waves(head_dim: int) -> int:
    return 8 if head_dim <= 128 else 4


def _wave_window_fits(span_tokens: int, page_size: int, head_dim: int) -> bool:
    """Whether each workgroup wave's share of span_tokens (whole 32-token steps
    from a step boundary) touches at most 64 pages (one table entry per lane)."""
    waves = _workgroup_waves(head_dim)
    wave_tokens = -(-(-(-span_tokens // 32)) // waves) * 32
    return (wave_tokens - 1) // page_size + 2 <= 64


def single_split_fits(capacity_tokens: int, page_size: int, head_dim: int) -> bool:
    """Whether one split covering the capacity runs the workgroup kernel (8
    waves, 4 above head_dim 128, per sequence and head group): pages of a
    multiple of 32 tokens, and every wave's share of the capacity's 32-token
    steps within 64 pages."""
    return page_size % 32 == 0 and _wave_window_fits(capacity_tokens, page_size, head_dim)


def takes_workgroup_splits(units: int, split_tokens: int, max_splits: int, page_size: int,
                           head_dim: int, capacity_tokens: int) -> bool:
    """The library's choice between one workgroup per split and one wave per
    split (mirrors lc_paged_decode_fwd): workgroups for a single split, splits
    of >= 2048 tokens, or grids of <= 512 splits."""
    span = capacity_tokens if max_splits == 1 else split_tokens
    return (page_size % 32 == 0 and _wave_window_fits(span, page_size, head_dim)
            and (max_splits == 1 or split_tokens >= 2048 or units * max_splits <= 512))


def choose_split_tokens(batch: int, n_kv_heads: int, group: int, capacity_tokens: int,
                        page_size: int = 64, head_dim: int = 128,
                        uniform_length: int | None = None, n_cus: int = 256) -> int:
    """Tokens per split.

    units = batch x kv heads x groups of <= 16 query heads. Where the page
    size allows workgroup splits (a multiple of 32 tokens):
      * uniform_length given (every sequence holds that many tokens, as in a
        batched decode step): the fewest splits per unit s whose units * s
        fill whole rounds of the CUs to >= 90%, each split a 1/s share of the
        length; s = 1 is one split over the capacity. Measured: config 4
        (256 units) 43.6 us against 46.0 us for 512-token splits; config 5
        (64 units x 4 splits of 8256) 168.9 us against 174.8 us at 2048.
      * lengths unknown (ragged), >= n_cus units and at most 256 sequences
        (the library then runs the splits longest first): s = 6 * n_cus /
        units splits per unit (rounded up), each a 1/s share of the capacity
        rounded up to 1024 tokens, at least 2048, more splits where a wave's
        share would touch over 64 pages. Measured on three seeds of config 2's
        length distribution (512 units, capacity 8192): 2816-4096-token
        splits within 1.5% of each other and 2-4% faster than 2048 (seed 0,
        the benchmark's: 180.2 us at 3072 against 187.1 us at 2048).
      * lengths unknown, more sequences: about 8 splits per CU for >= n_cus
        units (192 us at 2048-token splits against 197 us at 512 on config
        2's shape); one round of the CUs for fewer units, whatever the batch
        (16 sequences of 1-16K tokens, 128 units: 115.7 us at 8192 against
        127-133 us at 512-2048).
    Where the library would run such a split size with one wave per split
    instead (see takes_workgroup_splits), or pages are not a multiple of 32,
    one-wave splits: 512 tokens, shrunk until there are >= 1024 of them.
    """
    units = batch * n_kv_heads * ((group + 15) // 16)
    if units == 0:  # an empty batch launches nothing; any valid split will do
        return max(64, -(-capacity_tokens // 64) * 64)
    if page_size % 32 == 0 and capacity_tokens > 0:
        if uniform_length is not None:
            length = max(1, min(int(uniform_length), capacity_tokens))
            s = 1
            while s < 64:
                n = units * s
                if n >= n_cus and n / (n_cus * -(-n // n_cus)) >= 0.9:
                    break
                s += 1
            split = -(-(-(-length // s)) // 64) * 64
        elif units >= n_cus and batch <= 256:
            s = -(-6 * n_cus // units)
            while True:
                split = max(2048, -(-(-(-capacity_tokens // s)) // 1024) * 1024)
                if s >= 64 or _wave_window_fits(split, page_size, head_dim):
                    break
                s += 1
        elif units >= n_cus:
            s = -(-8 * n_cus // units)
            split = -(-(-(-capacity_tokens // s)) // 64) * 64
        else:
            s = max(1, n_cus // units)
            split = -(-(-(-capacity_tokens // s)) // 64) * 64
        if s == 1 or split >= capacity_tokens:
            split = -(-capacity_tokens // 64) * 64
        max_splits = -(-capacity_tokens // split)
        if takes_workgroup_splits(units, split, max_splits, page_size, head_dim,
                                  capacity_tokens):
            return split

    def n_splits(split: int) -> int:
        return units * ((capacity_tokens + split - 1) // split)

    split = 512
    while split > 64 and n_splits(split) < 1024:
        split //= 2
    return split


def paged_decode(q: torch.Tensor, key_pages: torch.Tensor, value_pages: torch.Tensor,
                 block_table: torch.Tensor, seq_lens: torch.Tensor, scale: float | None = None,
                 return_lse: bool = False, split_tokens: int | None = None,
                 workspace: torch.Tensor | None = None,
                 attention_mask: torch.Tensor | None = None, uniform_length: int | None = None):
    """One-token GQA attention per sequence over a paged K/V pool (forward only).

    q: [B, Hq, 1, D] or [B, Hq, D]; key_pages, value_pages: [N, Hkv, P, D];
    block_table: int32 [B, max_pages]; seq_lens: int32 [B]. attention_mask:
    additive scores for the query token, broadcastable to [B, Hq, 1, L] (or
    [B, Hq, L]); token t < L of a sequence gets mask[..., t], later tokens
    none. uniform_length: every seq_lens entry is known to equal this (a hint
    for the split choice only; results do not depend on it). Returns out with
    q's shape (and lse [B, Hq] fp32 if return_lse).
    """
    args = (block_table, seq_lens, scale, return_lse, split_tokens, workspace, attention_mask,
            uniform_length)
    if _records_grad(q, key_pages, value_pages):
        return _ForwardOnly.apply("paged_decode", lambda a, k, v: _paged_decode(a, k, v, *args),
                                  q, key_pages, value_pages)
    return _paged_decode(q, key_pages, value_pages, *args)


def _paged_decode(q: torch.Tensor, key_pages: torch.Tensor, value_pages: torch.Tensor,
                  block_table: torch.Tensor, seq_lens: torch.Tensor, scale: float | None,
                  return_lse: bool, split_tokens: int | None, workspace: torch.Tensor | None,
                  attention_mask: torch.Tensor | None = None, uniform_length: int | None = None):
    squeeze = q.dim() == 3
    q4 = q.unsqueeze(2) if squeeze else q
    if q4.dim() != 4 or q4.shape[2] != 1:
        raise ValueError(f"q must be [batch, heads, 1, head_dim], got {tuple(q.shape)}")
    if key_pages.dim() != 4 or key_pages.shape != value_pages.shape:
        raise ValueError("key_pages and value_pages must both be [num_pages, kv_heads, page, dim]")
    if key_pages.stride() != value_pages.stride():
        value_pages = value_pages.contiguous()
        key_pages = key_pages.contiguous()
    B, Hq, _, D = q4.shape
    N, Hkv, P, Dk = key_pages.shape
    if Dk != D:
        raise ValueError(f"head_dim mismatch: q {D}, pages {Dk}")
    if Hkv == 0 or Hq % Hkv != 0:
        raise ValueError(f"n_heads ({Hq}) must be a multiple of n_kv_heads ({Hkv})")
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise TypeError("block_table and seq_lens must be int32")
    if block_table.dim() != 2 or block_table.shape[0] != B or seq_lens.shape != (B,):
        raise ValueError("block_table must be [batch, max_pages] and seq_lens [batch]")
    if q4.dtype != key_pages.dtype or q4.dtype != value_pages.dtype:
        raise TypeError("q and the page pools must share a dtype")
    dev = nat.require_device(q4, key_pages, value_pages, block_table, seq_lens)
    if q4.stride(-1) != 1:
        q4 = q4.contiguous()
    if key_pages.stride(-1) != 1:
        key_pages = key_pages.contiguous()
        value_pages = value_pages.contiguous()
    if block_table.stride(-1) != 1:
        block_table = block_table.contiguous()
    if not seq_lens.is_contiguous():
        seq_lens = seq_lens.contiguous()
    if B == 0:
        out = torch.empty_like(q)
        return (out, torch.empty(0, Hq, dtype=torch.float32, device=dev)) if return_lse else out
    maxp = block_table.shape[1]
    capacity = maxp * P
    G = Hq // Hkv
    if split_tokens is None:
        split_tokens = choose_split_tokens(B, Hkv, G, capacity, P, D, uniform_length,
                                           _cu_count(dev))
    max_splits = max(1, (capacity + split_tokens - 1) // split_tokens)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lib = nat.load()
    need = lib.lc_paged_decode_workspace_bytes(B, Hq, D, max_splits)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    bias = None
    if attention_mask is not None:
        nat.require_device(q4, attention_mask)
        bias = decode_bias(attention_mask, B, Hq, q4.dtype)
    out = torch.empty((B, Hq, 1, D), dtype=q4.dtype, device=dev)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=dev) if return_lse else None
    # The ticket of the longest-first order's dynamic tail (zero-on-exit); a
    # capture before any eager call runs the static order (no counters).
    counters = _zeroed_counters("paged_decode", dev, lib.lc_paged_decode_counter_count(),
                                optional=True)
    with _DeviceGuard(dev):
        rc = lib.lc_paged_decode_fwd(
            q4.data_ptr(), q4.stride(0), q4.stride(1), key_pages.data_ptr(),
            value_pages.data_ptr(), key_pages.stride(0), key_pages.stride(1),
            key_pages.stride(2), block_table.data_ptr(), block_table.stride(0), maxp, N,
            seq_lens.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
            None if lse is None else lse.data_ptr(),
            None if bias is None else bias.data_ptr(), 0 if bias is None else bias.stride(0),
            0 if bias is None else bias.stride(1), 0 if bias is None else bias.shape[-1],
            0 if bias is None else nat.lc_dtype(bias), workspace.data_ptr(),
            workspace.numel() * workspace.element_size(),
            None if counters is None else counters.data_ptr(), B, Hq, Hkv, D, P,
            split_tokens, max_splits, float(scale), nat.lc_dtype(q4), _stream(dev))
    nat.check(rc, "lc_paged_decode_fwd")
    if squeeze:
        out = out.squeeze(2)
    return (out, lse) if return_lse else out


# ---------------------------------------------------------------------------
# Page-pool append / gather  (reference: models/llama3/kv_cache.py:38-83)
# ---------------------------------------------------------------------------
def _pool_checks(key_pages, value_pages, block_table):
    if key_pages.dim() != 4 or key_pages.shape != value_pages.shape:
        raise ValueError("page pools must both be [num_pages, kv_heads, page, dim]")
    if key_pages.stride() != value_pages.stride() or key_pages.stride(-1) != 1:
        raise ValueError("key_pages and value_pages must share a layout with unit dim stride")
    if block_table.dtype != torch.int32 or block_table.dim() != 2:
        raise TypeError("block_table must be int32 [batch, max_pages]")
    if block_table.stride(-1) != 1:
        raise ValueError("block_table rows must be contiguous")


def kv_append(k_new: torch.Tensor, v_new: torch.Tensor, key_pages: torch.Tensor,
              value_pages: torch.Tensor, block_table: torch.Tensor,
              start_pos: torch.Tensor) -> None:
    """Write k_new/v_new [B, Hkv, S, D] at positions start_pos[b] + s."""
    _pool_checks(key_pages, value_pages, block_table)
    if k_new.shape != v_new.shape or k_new.dim() != 4:
        raise ValueError("k_new and v_new must both be [batch, kv_heads, seq, head_dim]")
    B, Hkv, S, D = k_new.shape
    N, Hp, P, Dp = key_pages.shape
    if Hp != Hkv or Dp != D or block_table.shape[0] != B:
        raise ValueError("new tokens do not match the cache layout")
    if start_pos.dtype != torch.int32 or start_pos.shape != (B,):
        raise TypeError("start_pos must be int32 [batch]")
    if k_new.dtype != key_pages.dtype or v_new.dtype != key_pages.dtype:
        raise TypeError("new tokens must have the cache dtype")
    dev = nat.require_device(k_new, v_new, key_pages, value_pages, block_table, start_pos)
    if k_new.stride(-1) != 1:
        k_new = k_new.contiguous()
    if v_new.stride(-1) != 1:
        v_new = v_new.contiguous()
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_paged_kv_append(
            k_new.data_ptr(), v_new.data_ptr(), _i64arr(k_new.stride()), _i64arr(v_new.stride()),
            key_pages.data_ptr(), value_pages.data_ptr(), key_pages.stride(0),
            key_pages.stride(1), key_pages.stride(2), block_table.data_ptr(),
            block_table.stride(0), block_table.shape[1], N, start_pos.data_ptr(), B, Hkv, S, D,
            P, nat.lc_dtype(k_new), _stream(dev))
    nat.check(rc, "lc_paged_kv_append")


def rope_kv_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                   sin: torch.Tensor, key_pages: torch.Tensor, value_pages: torch.Tensor,
                   block_table: torch.Tensor, seq_lens: torch.Tensor) -> torch.Tensor:
    """Decode-time RoPE + cache append in one launch.

    Rotates q and k at positions seq_lens[b] + s (cos/sin: full tables indexed
    by position, covering the block-table capacity), writes the rotated k and
    v into the page pools, advances seq_lens by S in place and returns the
    rotated q as a new contiguous [B, Hq, S, D] tensor. Forward only.
    """
    if _records_grad(q, k, v):
        return _ForwardOnly.apply(
            "rope_kv_append",
            lambda a, b, c: _rope_kv_append(a, b, c, cos, sin, key_pages, value_pages,
                                            block_table, seq_lens), q, k, v)
    return _rope_kv_append(q, k, v, cos, sin, key_pages, value_pages, block_table, seq_lens)


def _rope_kv_append(q, k, v, cos, sin, key_pages, value_pages, block_table, seq_lens):
    _pool_checks(key_pages, value_pages, block_table)
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        raise ValueError("q must be [B, Hq, S, D] and k, v [B, Hkv, S, D]")
    B, Hq, S, D = q.shape
    N, Hkv, P, Dp = key_pages.shape
    if k.shape != (B, Hkv, S, D) or Dp != D or block_table.shape[0] != B:
        raise ValueError("q/k/v do not match the cache layout")
    if seq_lens.dtype != torch.int32 or seq_lens.shape != (B,):
        raise TypeError("seq_lens must be int32 [batch]")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != D:
        raise ValueError("cos/sin must be [positions, head_dim]")
    if not (q.dtype == k.dtype == v.dtype == cos.dtype == sin.dtype == key_pages.dtype):
        raise TypeError("q, k, v, cos, sin and the pools must share a dtype")
    dev = nat.require_device(q, k, v, cos, sin, key_pages, value_pages, block_table, seq_lens)
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    cos = cos if cos.stride(-1) == 1 else cos.contiguous()
    sin = sin if sin.stride(-1) == 1 else sin.contiguous()
    q_out = torch.empty((B, Hq, S, D), dtype=q.dtype, device=dev)
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_rope_kv_append(
            q.data_ptr(), _i64arr(q.stride()), k.data_ptr(), _i64arr(k.stride()), v.data_ptr(),
            _i64arr(v.stride()), q_out.data_ptr(), _i64arr(q_out.stride()), cos.data_ptr(),
            sin.data_ptr(), cos.stride(0), sin.stride(0), cos.shape[0], key_pages.data_ptr(),
            value_pages.data_ptr(), key_pages.stride(0), key_pages.stride(1), key_pages.stride(2),
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1], N,
            seq_lens.data_ptr(), B, Hq, Hkv, S, D, P, nat.lc_dtype(q), _stream(dev))
    nat.check(rc, "lc_rope_kv_append")
    return q_out


def decode_step_supported(dtype: torch.dtype, head_dim: int, page_size: int,
                          capacity_tokens: int) -> bool:
    """Whether lc_paged_decode_step takes these sizes (bf16/f16, head_dim a
    multiple of 16 up to 256, and the single-split kernel's page rule)."""
    return (dtype in (torch.bfloat16, torch.float16) and head_dim % 16 == 0
            and 16 <= head_dim <= 256
            and single_split_fits(capacity_tokens, page_size, head_dim))


def paged_decode_step(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                      sin: torch.Tensor, key_pages: torch.Tensor, value_pages: torch.Tensor,
                      block_table: torch.Tensor, seq_lens: torch.Tensor, counters: torch.Tensor,
                      scale: float | None = None, attention_mask: torch.Tensor | None = None,
                      return_lse: bool = False):
    """RoPE of the new token at p = seq_lens[b], its append to the page pools and
    decode attention over the cache including it, in one launch; seq_lens
    advances by one in place.

    q [B, Hq, 1, D], k and v [B, Hkv, 1, D] (unrotated projections); cos/sin
    full tables indexed by position covering the block-table capacity;
    counters: int32 [B] zeros (left at zero). attention_mask as in
    paged_decode over token indices 0 .. p. Returns out [B, Hq, 1, D] (a view
    of a [B, 1, Hq, D] buffer) and lse [B, Hq] if return_lse. Forward only.
    """
    args = (cos, sin, key_pages, value_pages, block_table, seq_lens, counters, scale,
            attention_mask, return_lse)
    if _records_grad(q, k, v):
        return _ForwardOnly.apply("paged_decode_step",
                                  lambda a, b, c: _paged_decode_step(a, b, c, *args), q, k, v)
    return _paged_decode_step(q, k, v, *args)


def _paged_decode_step(q, k, v, cos, sin, key_pages, value_pages, block_table, seq_lens,
                       counters, scale, attention_mask, return_lse):
    _pool_checks(key_pages, value_pages, block_table)
    if q.dim() != 4 or k.dim() != 4 or k.shape != v.shape or q.shape[2] != 1:
        raise ValueError("q must be [B, Hq, 1, D] and k, v [B, Hkv, 1, D]")
    B, Hq, _, D = q.shape
    N, Hkv, P, Dp = key_pages.shape
    if k.shape != (B, Hkv, 1, D) or Dp != D or block_table.shape[0] != B:
        raise ValueError("q/k/v do not match the cache layout")
    if Hq % Hkv != 0:
        raise ValueError(f"n_heads ({Hq}) must be a multiple of n_kv_heads ({Hkv})")
    for name, t in (("seq_lens", seq_lens), ("counters", counters)):
        if t.dtype != torch.int32 or t.shape != (B,) or not t.is_contiguous():
            raise TypeError(f"{name} must be a contiguous int32 [batch] tensor")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != D:
        raise ValueError("cos/sin must be [positions, head_dim]")
    if not (q.dtype == k.dtype == v.dtype == cos.dtype == sin.dtype == key_pages.dtype):
        raise TypeError("q, k, v, cos, sin and the pools must share a dtype")
    capacity = block_table.shape[1] * P
    if not decode_step_supported(q.dtype, D, P, capacity):
        raise ValueError(
            f"the fused decode step takes bf16/f16, head_dim a multiple of 16 <= 256 and "
            f"page_size a multiple of 32 with a capacity the one-workgroup kernel covers; got "
            f"{q.dtype}, head_dim {D}, page_size {P}, capacity {capacity}")
    dev = nat.require_device(q, k, v, cos, sin, key_pages, value_pages, block_table, seq_lens,
                             counters)
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    cos = cos if cos.stride(-1) == 1 else cos.contiguous()
    sin = sin if sin.stride(-1) == 1 else sin.contiguous()
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    bias = None
    if attention_mask is not None:
        nat.require_device(q, attention_mask)
        bias = decode_bias(attention_mask, B, Hq, q.dtype)
    buf = torch.empty((B, 1, Hq, D), dtype=q.dtype, device=dev)
    out = buf.transpose(1, 2)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=dev) if return_lse else None
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_paged_decode_step(
            q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1), cos.data_ptr(), sin.data_ptr(),
            cos.stride(0), sin.stride(0), cos.shape[0], key_pages.data_ptr(),
            value_pages.data_ptr(), key_pages.stride(0), key_pages.stride(1), key_pages.stride(2),
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1], N,
            seq_lens.data_ptr(), counters.data_ptr(), out.data_ptr(), out.stride(0),
            out.stride(1), None if lse is None else lse.data_ptr(),
            None if bias is None else bias.data_ptr(), 0 if bias is None else bias.stride(0),
            0 if bias is None else bias.stride(1), 0 if bias is None else bias.shape[-1],
            0 if bias is None else nat.lc_dtype(bias), B, Hq, Hkv, D, P, float(scale),
            nat.lc_dtype(q), _stream(dev))
    nat.check(rc, "lc_paged_decode_step")
    return (out, lse) if return_lse else out


def kv_gather(key_pages: torch.Tensor, value_pages: torch.Tensor, block_table: torch.Tensor,
              length: int):
    """Contiguous [B, Hkv, length, D] copies of the first `length` tokens."""
    _pool_checks(key_pages, value_pages, block_table)
    N, Hkv, P, D = key_pages.shape
    B = block_table.shape[0]
    if length > block_table.shape[1] * P:
        raise ValueError("length exceeds the block-table capacity")
    dev = nat.require_device(key_pages, value_pages, block_table)
    k_out = torch.empty((B, Hkv, length, D), dtype=key_pages.dtype, device=dev)
    v_out = torch.empty_like(k_out)
    lib = nat.load()
    with _DeviceGuard(dev):
        rc = lib.lc_paged_kv_gather(
            key_pages.data_ptr(), value_pages.data_ptr(), key_pages.stride(0),
            key_pages.stride(1), key_pages.stride(2), block_table.data_ptr(),
            block_table.stride(0), block_table.shape[1], N, k_out.data_ptr(), v_out.data_ptr(),
            B, Hkv, length, D, P, nat.lc_dtype(key_pages), _stream(dev))
    nat.check(rc, "lc_paged_kv_gather")
    return k_out, v_out
