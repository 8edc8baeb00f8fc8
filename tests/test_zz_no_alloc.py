"""GPU test of lc_paged_decode_fwd_noalloc, the allocation-free decode entry.

It must produce exactly what lc_paged_decode_fwd produces with a caller
workspace (same kernels, same split configuration, so bit-identical outputs
and logsumexps), meet the oracle's bar, do so on two calls in a row with the
second one smaller (the device scratch keeps the first call's contents), and
reject a request whose split partials exceed the fixed scratch before any
launch.
"""
import math

import pytest
import torch

from helpers import ATOL, assert_close, assert_lse_close
from oracle.decode import paged_decode

pytestmark = pytest.mark.gpu

LC_EWORKSPACE = -3


def _case(lens, Hq, Hkv, D, P, seed):
    g = torch.Generator().manual_seed(seed)
    pages = [max(1, math.ceil(n / P)) for n in lens]
    N = sum(pages) + 2
    perm = torch.randperm(N, generator=g).to(torch.int32)
    bt = torch.full((len(lens), max(pages)), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[o:o + n]
        o += n
    kp = torch.randn(N, Hkv, P, D, generator=g).bfloat16()
    vp = torch.randn(N, Hkv, P, D, generator=g).bfloat16()
    q = torch.randn(len(lens), Hq, 1, D, generator=g).bfloat16()
    return q, kp, vp, bt, torch.tensor(lens, dtype=torch.int32)


def _noalloc(lib, q, kp, vp, bt, sl, split, max_splits):
    from llm_cuda import _native

    B, Hq, _, D = q.shape
    N, Hkv, P, _ = kp.shape
    out = torch.full((B, Hq, 1, D), float("nan"), dtype=q.dtype, device=q.device)
    lse = torch.full((B, Hq), float("nan"), dtype=torch.float32, device=q.device)
    rc = lib.lc_paged_decode_fwd_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(), kp.stride(0),
        kp.stride(1), kp.stride(2), bt.data_ptr(), bt.stride(0), bt.shape[1], N, sl.data_ptr(),
        out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(), None, 0, 0, 0, 0, B, Hq,
        Hkv, D, P, split, max_splits, 1.0 / math.sqrt(D), _native.lc_dtype(q),
        torch.cuda.current_stream().cuda_stream)
    _native.check(rc, "lc_paged_decode_fwd_noalloc")
    return out, lse


@pytest.mark.parametrize("second", [
    dict(lens=[700, 5, 1030], Hq=32, Hkv=8, D=128, P=64),   # smaller batch, same layout
    dict(lens=[3, 300], Hq=8, Hkv=2, D=64, P=16),           # smaller still, per-lane-page kernel
])
def test_noalloc_matches_workspace_entry_twice(cuda, second):
    from llm_cuda import _native
    from llm_cuda.kernels import _ops

    lib = _native.load()
    first = dict(lens=[4100, 64, 2999, 8000, 513, 1, 6000, 2048], Hq=32, Hkv=8, D=128, P=64)
    for call, spec in enumerate((first, second)):
        q, kp, vp, bt, sl = _case(spec["lens"], spec["Hq"], spec["Hkv"], spec["D"], spec["P"],
                                  seed=40 + call)
        dq, dkp, dvp, dbt, dsl = (t.to(cuda) for t in (q, kp, vp, bt, sl))
        B, Hq, Hkv = len(spec["lens"]), spec["Hq"], spec["Hkv"]
        cap = bt.shape[1] * spec["P"]
        split = _ops.choose_split_tokens(B, Hkv, Hq // Hkv, cap)
        max_splits = max(1, math.ceil(cap / split))
        need = lib.lc_paged_decode_workspace_bytes(B, Hq, spec["D"], max_splits)
        assert 0 < need <= 32 << 20
        ref_out, ref_lse = _ops.paged_decode(dq, dkp, dvp, dbt, dsl, return_lse=True,
                                             split_tokens=split)
        out, lse = _noalloc(lib, dq, dkp, dvp, dbt, dsl, split, max_splits)
        torch.cuda.synchronize()
        print(f"call {call}: B={B} Hq={Hq} D={spec['D']} P={spec['P']} split={split} "
              f"splits={max_splits} scratch bytes={need}", flush=True)
        assert torch.equal(out, ref_out), f"call {call}: output differs from the workspace entry"
        assert torch.equal(lse, ref_lse), f"call {call}: lse differs from the workspace entry"
        o_ref, l_ref = paged_decode(q, kp, vp, bt, sl)
        assert_close(out, o_ref, ATOL[torch.bfloat16], f"call {call} vs oracle")
        assert_lse_close(lse, l_ref)


def test_noalloc_rejects_partials_beyond_the_scratch(cuda):
    """64 sequences x 64 heads x 512 splits x head_dim 128 needs 1 GiB of
    partials: refused with LC_EWORKSPACE before anything is launched. Every
    argument is a real device buffer of the shape it claims (empty sequences
    over a one-page pool), so the call stays in bounds even if the size check
    ever ran after a launch."""
    from llm_cuda import _native

    lib = _native.load()
    B, Hq, Hkv, D, P, max_pages, split, max_splits = 64, 64, 8, 128, 64, 512, 64, 512
    assert lib.lc_paged_decode_workspace_bytes(B, Hq, D, max_splits) > 32 << 20
    q = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=cuda)
    kp = torch.zeros(1, Hkv, P, D, dtype=torch.bfloat16, device=cuda)
    vp = torch.zeros_like(kp)
    bt = torch.zeros(B, max_pages, dtype=torch.int32, device=cuda)
    sl = torch.zeros(B, dtype=torch.int32, device=cuda)
    out = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=cuda)
    lse = torch.zeros(B, Hq, dtype=torch.float32, device=cuda)
    rc = lib.lc_paged_decode_fwd_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(), kp.stride(0),
        kp.stride(1), kp.stride(2), bt.data_ptr(), bt.stride(0), max_pages, kp.shape[0],
        sl.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(), None, 0, 0,
        0, 0, B, Hq, Hkv, D, P, split, max_splits, 1.0, _native.lc_dtype(q),
        torch.cuda.current_stream().cuda_stream)
    assert rc == LC_EWORKSPACE
    assert b"scratch" in lib.lc_last_error()
    torch.cuda.synchronize()
    assert not out.any() and not lse.any(), "a rejected call wrote its outputs"
