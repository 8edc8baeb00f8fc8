"""Seeded random shapes for the attention, decode-step and lm_head kernels, against the oracle.

Each case draws its shape from a numpy generator seeded by the case number, so
the set is fixed and every failure names a reproducible case (the pytest id
carries the shape). Shapes stay small enough for the CPU oracle; they cover
what the hand-picked cases elsewhere fix only at chosen points: odd batch
sizes, group sizes 1-20, head_dims 64-256, page sizes 16-128 (and 48, not a
power of two), empty and one-token sequences, split sizes chosen by the
library or forced, cached-prefix offsets, vocabularies that are not tile
multiples.

Decode: out within the dtype's atol and lse within 1e-3 relative of
oracle.decode.paged_decode; pools poisoned with NaN outside the sequences'
slots (a stray read shows up as NaN); a second call equal bit for bit.
Fused decode step: pools and lengths bit-identical to RoPE + append, out and
lse against the oracle's decode over the advanced lengths (the rule of
tests/test_gpu_decode_step.py), positions past the capacity included.
Prefill: oracle.attention.causal_attention with the same q_offset; backward:
oracle.attention.causal_attention_backward (the bound of
tests/test_gpu_prefill_bwd.py).
lm_head + argmax: the ids rule of tests/test_gpu_lm_head.py (one ulp of slack
at a rounding boundary, at most one such row).
Elementwise (RMSNorm, add + RMSNorm, SwiGLU, RoPE): random widths (odd ones
take the element-wise path), rows taken from wider buffers at random offsets
(strided, possibly unaligned), fp32/f16/bf16, against oracle.elementwise with
the bounds of tests/test_gpu_elementwise.py; the residual sum bit-exact.
"""
import numpy as np
import pytest
import torch

from helpers import ATOL, RTOL, assert_close, assert_lse_close
from oracle.attention import causal_attention
from oracle.decode import paged_decode
from oracle.elementwise import apply_rope, rms_norm, swiglu
from test_gpu_decode import _paged_case
from test_gpu_decode_step import _case as _step_case, _check as _check_step
from test_gpu_decode_step import _fused as _step_fused, _unfused as _step_unfused
from test_gpu_lm_head import _check as _check_lm_head
from test_gpu_prefill_bwd import _check as _check_bwd, _inputs as _bwd_inputs

pytestmark = pytest.mark.gpu


def _decode_case(i):
    r = np.random.default_rng(1000 + i)
    dtype = torch.float16 if r.random() < 0.3 else torch.bfloat16
    Hkv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 3, 4, 8, 16]))
    D = int(r.choice([64, 96, 128, 128, 256]))
    P = int(r.choice([16, 32, 48, 64, 64, 128]))
    B = int(r.integers(1, 81))
    lmax = int(r.choice([64, 700, 3000, 6000]))
    # bound the pools (and the oracle's work): tokens x Hkv x D <= 2^25
    lmax = max(1, min(lmax, (1 << 25) // (B * Hkv * D)))
    lens = r.integers(0, lmax + 1, B)
    lens[r.random(B) < 0.1] = 0
    if B > 2:
        lens[int(r.integers(0, B))] = 1
    split = None if r.random() < 0.5 else int(r.choice([64, 256, 512, 1024, 2048, 3072]))
    return dict(lens=[int(x) for x in lens], Hq=Hkv * G, Hkv=Hkv, D=D, P=P, dtype=dtype,
                split=split)


def _prefill_case(i):
    r = np.random.default_rng(2000 + i)
    dtype = torch.float16 if r.random() < 0.3 else torch.bfloat16
    Hkv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 4, 8]))
    D = int(r.choice([64, 128, 128]))
    B = int(r.integers(1, 4))
    Sq = int(r.integers(1, 600))
    off = 0 if r.random() < 0.5 else int(r.integers(1, 300))
    # bound the oracle's work: B x Hq x Sq x Skv x D <= 2^31
    while B * Hkv * G * Sq * (Sq + off) * D > (1 << 31) and Sq > 1:
        Sq //= 2
    return dict(B=B, Hq=Hkv * G, Hkv=Hkv, Sq=Sq, off=off, D=D, dtype=dtype)


def _step_case_params(i):
    r = np.random.default_rng(4000 + i)
    dtype = torch.float16 if r.random() < 0.3 else torch.bfloat16
    Hkv = int(r.choice([1, 2, 4, 8]))
    G = int(r.choice([1, 2, 4, 5, 8, 20]))
    D = int(r.choice([64, 96, 128, 128, 256]))
    P = int(r.choice([32, 64, 128]))
    maxp = int(r.integers(1, 21))
    B = int(r.integers(1, 49))
    cap = maxp * P
    lens = r.integers(0, cap + 1, B)
    if B > 3:  # one past the capacity (dropped), one at the last slot, one empty
        lens[:3] = [cap + int(r.integers(0, 100)), cap - 1, 0]
    return dict(lens=[int(x) for x in lens], Hq=Hkv * G, Hkv=Hkv, D=D, P=P, maxp=maxp,
                dtype=dtype)


def _bwd_case(i):
    r = np.random.default_rng(5000 + i)
    dtype = torch.float16 if r.random() < 0.3 else torch.bfloat16
    Hkv = int(r.choice([1, 2, 4]))
    G = int(r.choice([1, 2, 4]))
    D = int(r.choice([64, 128]))
    B = int(r.integers(1, 3))
    Sq = int(r.integers(1, 300))
    off = 0 if r.random() < 0.5 else int(r.integers(1, 200))
    return dict(B=B, Hq=Hkv * G, Hkv=Hkv, Sq=Sq, off=off, D=D, dtype=dtype)


def _lm_head_case(i):
    r = np.random.default_rng(3000 + i)
    dtype = torch.float16 if r.random() < 0.3 else torch.bfloat16
    B = int(r.integers(1, 71))
    K = int(r.choice([128, 256, 384, 512, 1024, 4096]))
    V = int(r.integers(2, 30001))
    V = max(2, min(V, (1 << 25) // K))
    return dict(B=B, K=K, V=V, dtype=dtype)


def _ew_case(i):
    r = np.random.default_rng(6000 + i)
    dtype = [torch.float32, torch.float16, torch.bfloat16][int(r.integers(0, 3))]
    kind = ["rmsnorm", "add_rmsnorm", "swiglu", "rope"][i % 4]
    rows = int(r.integers(1, 40))
    width = int(r.choice([16, 100, 256, 1001, 4096, 5000, 14336, 20480]))
    if kind == "rope":
        width = int(r.choice([16, 32, 64, 96, 128, 256]))  # head_dim
    pad = int(r.choice([0, 0, 8, 3]))  # row stride width + pad, rows start at offset pad
    return dict(kind=kind, rows=rows, width=width, pad=pad, dtype=dtype)


_DT = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def _id(case):
    return "-".join(f"{k}{v}" if k != "lens" else f"B{len(v)}max{max(v)}"
                    for k, v in case.items() if k != "dtype") + "-" + _DT[case["dtype"]]


DECODE = [_decode_case(i) for i in range(24)]
PREFILL = [_prefill_case(i) for i in range(16)]
LM_HEAD = [_lm_head_case(i) for i in range(16)]
STEP = [_step_case_params(i) for i in range(12)]
ELEMENTWISE = [_ew_case(i) for i in range(24)]
BWD = [_bwd_case(i) for i in range(10)]


@pytest.mark.parametrize("case", DECODE, ids=[_id(c) for c in DECODE])
def test_fuzz_paged_decode(cuda, case):
    from llm_cuda.kernels.triton.decode_attention import paged_decode_attention

    c = case
    q, kp, vp, bt, sl = _paged_case(c["lens"], c["Hq"], c["Hkv"], c["D"], c["P"], c["dtype"],
                                    cuda, seed=len(c["lens"]), poison=True)
    kw = {} if c["split"] is None else {"split_tokens": c["split"]}
    dev = [t.to(cuda) for t in (q, kp, vp, bt, sl)]
    out, lse = paged_decode_attention(*dev, return_lse=True, **kw)
    out2, lse2 = paged_decode_attention(*dev, return_lse=True, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out, out2) and torch.equal(lse, lse2), "second call differs"
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert_close(out, ref, ATOL[c["dtype"]], f"decode {_id(c)}")
    assert_lse_close(lse, ref_lse, f"decode lse {_id(c)}")


@pytest.mark.parametrize("case", PREFILL, ids=[_id(c) for c in PREFILL])
def test_fuzz_prefill(cuda, case):
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention

    c = case
    g = torch.Generator().manual_seed(c["Sq"] * 31 + c["off"])
    Skv = c["Sq"] + c["off"]
    q = torch.randn(c["B"], c["Hq"], c["Sq"], c["D"], generator=g).to(c["dtype"])
    k = torch.randn(c["B"], c["Hkv"], Skv, c["D"], generator=g).to(c["dtype"])
    v = torch.randn(c["B"], c["Hkv"], Skv, c["D"], generator=g).to(c["dtype"])
    out, lse = triton_fused_causal_attention(q.to(cuda), k.to(cuda), v.to(cuda),
                                             return_lse=True, q_offset=c["off"])
    ref, ref_lse = causal_attention(q, k, v, q_offset=c["off"])
    assert_close(out, ref, ATOL[c["dtype"]], f"prefill {_id(c)}")
    assert_lse_close(lse, ref_lse, f"prefill lse {_id(c)}")


@pytest.mark.parametrize("case", LM_HEAD, ids=[_id(c) for c in LM_HEAD])
def test_fuzz_lm_head_argmax(cuda, case):
    c = case
    g = torch.Generator().manual_seed(c["V"] + c["K"])
    hidden = torch.randn(c["B"], c["K"], generator=g).to(c["dtype"]).to(cuda)
    weight = (torch.randn(c["V"], c["K"], generator=g) * 0.02).to(c["dtype"]).to(cuda)
    _check_lm_head(hidden, weight, max_mismatch=1)


@pytest.mark.parametrize("case", STEP, ids=[_id(c) for c in STEP])
def test_fuzz_decode_step(cuda, case):
    c = case
    args = _step_case(c["lens"], c["Hq"], c["Hkv"], c["D"], c["P"], c["maxp"], c["dtype"], cuda,
                      seed=len(c["lens"]) + c["D"])
    _check_step(_step_fused(*args), _step_unfused(*args), c["dtype"], f"step {_id(c)}")


@pytest.mark.parametrize("case", BWD, ids=[_id(c) for c in BWD])
def test_fuzz_prefill_backward(cuda, case):
    c = case
    q, k, v, do = _bwd_inputs(c["B"], c["Hq"], c["Hkv"], c["Sq"], c["Sq"] + c["off"], c["D"],
                              c["dtype"], cuda, seed=c["Sq"] * 7 + c["off"])
    _check_bwd(q, k, v, do, c["off"], c["dtype"])


@pytest.mark.parametrize("case", ELEMENTWISE, ids=[_id(c) for c in ELEMENTWISE])
def test_fuzz_elementwise(cuda, case):
    from llm_cuda.kernels import _ops

    c = case
    dt, rows, n, pad = c["dtype"], c["rows"], c["width"], c["pad"]
    g = torch.Generator().manual_seed(rows * 131 + n + pad)
    tol, rtol = ATOL[dt], RTOL[dt]

    def strided(cols):  # rows x cols inside a [rows, cols + pad] buffer, from column pad
        base = torch.randn(rows, cols + 2 * pad, generator=g).to(dt).to(cuda)
        return base[:, pad:pad + cols]

    if c["kind"] in ("rmsnorm", "add_rmsnorm"):
        x, w = strided(n), (1 + 0.1 * torch.randn(n, generator=g)).to(dt).to(cuda)
        if c["kind"] == "rmsnorm":
            y = _ops.rms_norm(x, w, 1e-5)
            ref = rms_norm(x.cpu(), w.cpu(), 1e-5)
        else:
            res = strided(n)
            y, ssum = _ops.add_rms_norm(x, res, w, 1e-5)
            assert torch.equal(ssum, x + res), "residual sum"
            ref = rms_norm((x + res).cpu(), w.cpu(), 1e-5)
        assert_close(y, ref, tol, _id(c), rtol=rtol)
    elif c["kind"] == "swiglu":
        gate, up = strided(n), strided(n)
        gate.mul_(3)  # in place: the view keeps its strides
        assert_close(_ops.swiglu(gate, up), swiglu(gate.cpu(), up.cpu()), tol, _id(c), rtol=rtol)
    else:
        from llm_cuda.kernels.triton.rope import triton_apply_rope

        D, H, S = n, 1 + rows % 5, 1 + rows
        q = torch.randn(2, S, H * D + pad, generator=g).to(dt).to(cuda)[..., :H * D]
        q = q.view(2, S, H, D).transpose(1, 2)  # projection-view strides
        cos = torch.randn(S, D, generator=g).to(dt).to(cuda)  # full-width tables, unequal halves
        sin = torch.randn(S, D, generator=g).to(dt).to(cuda)
        out = triton_apply_rope(q, cos, sin)
        ref = apply_rope(q.cpu(), cos.cpu(), sin.cpu())
        assert_close(out, ref, tol, _id(c), rtol=rtol)
