"""GPU parity: split-K paged flash-decode (MFMA bf16/f16 kernel, generic fp32
kernel) and the contiguous triton_decode_attention entry vs the oracle.

Cases follow the reference's decode tests (test_triton_decode_attention.py:
187-302, seed 42: MHA/GQA fp32, fp16, bf16, kv_len 1, long kv 1024, head_dim
48, batch > 1) and add what paging brings: ragged lengths, random page
permutations, NaN-poisoned unused slots, invalid table entries, empty
sequences, page sizes that are not powers of two, split-count invariance, and
the benchmark shapes (8B: 32/8 heads, D 128, P 64; 70B: 64/8 heads).
"""
import math

import pytest
import torch

from helpers import ATOL, assert_close, assert_lse_close
from oracle.decode import decode_attention, paged_decode

pytestmark = pytest.mark.gpu


def _contig_case(bsz, n_heads, n_kv_heads, kv_len, head_dim, dtype, device):
    torch.manual_seed(42)
    q = torch.randn(bsz, n_heads, 1, head_dim, dtype=dtype, device=device)
    k = torch.randn(bsz, n_kv_heads, kv_len, head_dim, dtype=dtype, device=device)
    v = torch.randn(bsz, n_kv_heads, kv_len, head_dim, dtype=dtype, device=device)
    return q, k, v


@pytest.mark.parametrize(
    "bsz,n_heads,n_kv_heads,kv_len,head_dim,dtype",
    [
        (2, 4, 4, 64, 32, torch.float32),     # MHA fp32
        (2, 8, 4, 64, 32, torch.float32),     # GQA fp32
        (1, 16, 8, 128, 64, torch.float16),   # GQA fp16
        (1, 16, 8, 128, 64, torch.bfloat16),  # GQA bf16
        (1, 4, 2, 1, 16, torch.float32),      # kv_len 1
        (1, 8, 4, 1024, 64, torch.float32),   # long kv
        (1, 4, 2, 32, 48, torch.float32),     # head_dim 48
        (1, 4, 2, 32, 48, torch.bfloat16),    # head_dim 48 on MFMA (padded to 64)
        (4, 8, 4, 64, 32, torch.float32),     # batch 4
        (3, 32, 8, 300, 128, torch.bfloat16),  # 8B head layout, odd length
        (2, 64, 8, 200, 128, torch.bfloat16),  # 70B head layout
        (2, 40, 2, 77, 128, torch.bfloat16),   # G = 20 > 16: two head groups
        (2, 8, 8, 129, 256, torch.bfloat16),   # head_dim 256
    ],
)
def test_triton_decode_attention_matches_oracle(cuda, bsz, n_heads, n_kv_heads, kv_len, head_dim,
                                                dtype):
    from llm_cuda.kernels.triton.decode_attention import triton_decode_attention

    q, k, v = _contig_case(bsz, n_heads, n_kv_heads, kv_len, head_dim, dtype, cuda)
    out, lse = triton_decode_attention(q, k, v, return_lse=True)
    assert out.shape == q.shape and out.dtype == q.dtype
    ref, ref_lse = decode_attention(q.cpu(), k.cpu(), v.cpu())
    assert_close(out, ref, ATOL[dtype], "decode out")
    assert_lse_close(lse, ref_lse)


def _paged_case(lens, Hq, Hkv, D, P, dtype, device, seed=0, poison=True, extra_pages=3):
    g = torch.Generator().manual_seed(seed)
    pages_per = [max(1, math.ceil(L / P)) for L in lens]
    maxp = max(pages_per)
    N = sum(pages_per) + extra_pages
    perm = torch.randperm(N, generator=g).to(torch.int32)
    bt = torch.full((len(lens), maxp), -1, dtype=torch.int32)
    o = 0
    for b, n in enumerate(pages_per):
        bt[b, :n] = perm[o:o + n]
        o += n
    kp = torch.randn(N, Hkv, P, D, generator=g).to(dtype)
    vp = torch.randn(N, Hkv, P, D, generator=g).to(dtype)
    if poison:
        # NaN in every slot no sequence owns: a read of one shows up as NaN.
        owned = torch.zeros(N, P, dtype=torch.bool)
        for b, L in enumerate(lens):
            for t in range(L):
                owned[bt[b, t // P], t % P] = True
        free = (~owned)[:, None, :, None].expand_as(kp)
        kp[free] = float("nan")
        vp[free] = float("nan")
    q = torch.randn(len(lens), Hq, 1, D, generator=g).to(dtype)
    sl = torch.tensor(lens, dtype=torch.int32)
    return q, kp, vp, bt, sl


def _run_paged(q, kp, vp, bt, sl, device, **kw):
    from llm_cuda.kernels.triton.decode_attention import paged_decode_attention

    return paged_decode_attention(q.to(device), kp.to(device), vp.to(device), bt.to(device),
                                  sl.to(device), return_lse=True, **kw)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("P", [64, 16, 4, 48])
def test_paged_ragged_random_permutation(cuda, dtype, P):
    lens = [1, 5, 64, 65, 200, 513, 3]
    q, kp, vp, bt, sl = _paged_case(lens, 8, 2, 128, P, dtype, cuda, seed=P)
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert_close(out, ref, ATOL[dtype], f"paged P={P}")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("P", [16, 48])
@pytest.mark.parametrize("D", [64, 48])
def test_paged_lanes_kernel_small_head_dim_g4(cuda, dtype, P, D):
    """Page sizes that are not multiples of 32 take the per-lane-page kernel;
    head_dim <= 64 runs its 64-wide instance (a tighter register budget)."""
    lens = [1, 17, 64, 100, 333, 48]
    q, kp, vp, bt, sl = _paged_case(lens, 8, 2, D, P, dtype, cuda, seed=P + D)
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert_close(out, ref, ATOL[dtype], f"lanes P={P} D={D}")
    assert_lse_close(lse, ref_lse)


def test_paged_empty_sequence_and_invalid_entries(cuda):
    lens = [0, 70, 130]
    q, kp, vp, bt, sl = _paged_case(lens, 4, 1, 64, 64, torch.bfloat16, cuda, seed=3)
    # an out-of-range entry beyond each sequence's length is never read
    bt[1, 2:] = 10 ** 6
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert (out[0].float().cpu() == 0).all()
    assert torch.isinf(lse[0].cpu()).all()
    assert_close(out[1:], ref[1:], ATOL[torch.bfloat16], "paged invalid")
    assert_lse_close(lse[1:], ref_lse[1:])


def test_paged_invalid_entry_inside_length_is_skipped(cuda):
    """A bad page id inside the live range is not dereferenced; its tokens drop out."""
    lens = [192]
    q, kp, vp, bt, sl = _paged_case(lens, 4, 2, 64, 64, torch.bfloat16, cuda, seed=4, poison=False)
    good = bt.clone()
    bt[0, 1] = -5
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda)
    keep = [0, 2]
    kk = torch.cat([kp[int(good[0, i])] for i in keep], dim=1)[None]
    vv = torch.cat([vp[int(good[0, i])] for i in keep], dim=1)[None]
    ref, ref_lse = decode_attention(q, kk, vv)
    assert_close(out, ref, ATOL[torch.bfloat16], "skip invalid")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_split_count_invariance(cuda, dtype):
    lens = [1000, 4097, 257]
    q, kp, vp, bt, sl = _paged_case(lens, 32, 8, 128, 64, dtype, cuda, seed=5)
    outs = [_run_paged(q, kp, vp, bt, sl, cuda, split_tokens=s) for s in (64, 256, 1024, 4160)]
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    for out, lse in outs:
        assert_close(out, ref, ATOL[dtype], "split invariance")
        assert_lse_close(lse, ref_lse)


def test_decode_equals_last_prefill_row(cuda):
    """Cross-kernel invariant: decode of token t == row t of causal prefill."""
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention
    from llm_cuda.kernels.triton.decode_attention import triton_decode_attention

    torch.manual_seed(11)
    q = torch.randn(2, 8, 96, 64, device=cuda)
    k = torch.randn(2, 2, 96, 64, device=cuda)
    v = torch.randn(2, 2, 96, 64, device=cuda)
    full, lfull = triton_fused_causal_attention(q, k, v, return_lse=True)
    dec, ldec = triton_decode_attention(q[:, :, -1:].contiguous(), k, v, return_lse=True)
    assert_close(dec[:, :, 0], full[:, :, -1], 1e-5, "decode vs prefill")
    assert_lse_close(ldec, lfull[:, :, -1])


def test_baseline_8b_shape_subset(cuda):
    """Benchmark config 2 construction (seed 0, ctx ~ U[512, 8192], P 64, random
    permutation) on 8 sequences, checked against the oracle."""
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 8193, (8,), generator=g).tolist()
    q, kp, vp, bt, sl = _paged_case(lens, 32, 8, 128, 64, torch.bfloat16, cuda, seed=0, poison=True)
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert_close(out, ref, ATOL[torch.bfloat16], "8B subset")
    assert_lse_close(lse, ref_lse)


def test_baseline_70b_long_context_subset(cuda):
    """Benchmark config 5 head layout (64/8 heads, D 128) at context 32768 on 2 sequences."""
    lens = [32768, 32768 - 37]
    q, kp, vp, bt, sl = _paged_case(lens, 64, 8, 128, 64, torch.bfloat16, cuda, seed=1, poison=False)
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert_close(out, ref, ATOL[torch.bfloat16], "70B subset")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype,P,split,masked,B", [
    (torch.bfloat16, 64, 2048, False, 64),   # config 2's kernel: table window loaded with the length
    (torch.float16, 64, 3072, False, 64),
    (torch.bfloat16, 32, 2048, False, 64),   # splits over 64 pages: per-wave table loads
    (torch.bfloat16, 64, 2048, True, 64),    # additive key mask
    (torch.bfloat16, 64, 3072, False, 37),   # lanes past the batch hold no sequence
    (torch.bfloat16, 64, 3072, False, 150),  # three 64-lane chunks of sequences
])
def test_longest_first_order_matches_split_major(cuda, dtype, P, split, masked, B):
    """A ragged batch of at most 256 sequences whose split workgroups take more
    than one round of the CUs runs its (sequence, split) pairs longest first:
    the whole splits, then each sequence's final partial split by decreasing
    length. Every split is computed as in the split-major grid, so the output
    equals, bit for bit, the same sequences in a batch of 257 (which keeps the
    split-major grid), and matches the oracle. Lengths cover an empty
    sequence, one token, whole splits only (no partial split), equal
    remainders in different sequences (also across 64-sequence chunks) and the
    longest length; a batch of 37 leaves lanes of the ordering wave without a
    sequence, one of 150 spans three chunks."""
    from llm_cuda.kernels.triton.decode_attention import paged_decode_attention

    g = torch.Generator().manual_seed(P + split + B)
    lens = torch.randint(0, 6001, (B,), generator=g).tolist()
    lens[:8] = [0, 1, 31, split, 2 * split, split + 7, 2 * split + 7, 6000]
    lens[-3:] = [lens[3] + 5, 2 * split + 7, 1]  # ties across the batch's chunks
    n_ref = 257  # a batch this large keeps the split-major grid
    Hq, Hkv, D = 32, 8, 128
    q, kp, vp, bt, sl = _paged_case(lens + [100] * (n_ref - B), Hq, Hkv, D, P, dtype, cuda,
                                    seed=P + 3)
    mask = None
    if masked:
        mask = torch.randn(n_ref, 1, 1, 6000, generator=g)
        mask[9, ..., 500:900] = float("-inf")
        mask[10, ..., :3000] = -1e4
        mask = mask.to(dtype)
    kw = {"split_tokens": split}

    def run(n):
        m = None if mask is None else mask[:n].to(cuda)
        return paged_decode_attention(q[:n].to(cuda), kp.to(cuda), vp.to(cuda), bt[:n].to(cuda),
                                      sl[:n].to(cuda), return_lse=True, attention_mask=m, **kw)

    out_b, lse_b = run(B)
    out_ref, lse_ref = run(n_ref)
    assert torch.equal(out_b, out_ref[:B]), "longest-first order changed the output"
    assert torch.equal(lse_b, lse_ref[:B])
    ref, ref_lse = paged_decode(q[:B], kp, vp, bt[:B], sl[:B],
                                bias=None if mask is None else mask[:B, :, 0].float())
    assert_close(out_b, ref, ATOL[dtype], f"longest-first P={P} split={split} B={B}")
    assert_lse_close(lse_b, ref_lse)


def _abi_decode(q, kp, vp, bt, sl, split, counters):
    """lc_paged_decode_fwd through the C ABI with the given counters (None: the
    static longest-first order)."""
    from llm_cuda import _native
    from llm_cuda.kernels import _ops

    lib = _native.load()
    B, Hq, _, D = q.shape
    N, Hkv, P, _ = kp.shape
    maxp = bt.shape[1]
    max_splits = max(1, math.ceil(maxp * P / split))
    need = lib.lc_paged_decode_workspace_bytes(B, Hq, D, max_splits)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=q.device)
    out = torch.empty_like(q)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=q.device)
    rc = lib.lc_paged_decode_fwd(
        q.data_ptr(), q.stride(0), q.stride(1), kp.data_ptr(), vp.data_ptr(), kp.stride(0),
        kp.stride(1), kp.stride(2), bt.data_ptr(), bt.stride(0), maxp, N, sl.data_ptr(),
        out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(), None, 0, 0, 0, 0,
        ws.data_ptr(), ws.numel(), None if counters is None else counters.data_ptr(), B, Hq, Hkv,
        D, P, split, max_splits, 1.0 / math.sqrt(D), _native.lc_dtype(q), _ops._stream(q.device))
    _native.check(rc, "lc_paged_decode_fwd")
    return out, lse


@pytest.mark.parametrize("B,lo,hi,split", [
    (64, 512, 8192, 3072),   # the config-2 mix: many dead slots in the grid
    (37, 0, 6000, 2048),     # lanes past the batch, empty sequences
    (150, 1, 6000, 2048),    # three 64-sequence chunks
    (256, 2048, 2048, 1024),  # every slot live, equal splits: the spare pool is empty
])
def test_dynamic_tail_matches_static_order(cuda, B, lo, hi, split):
    """With counters, the last quarter of the longest-first ranks is handed out
    by a ticket in the order the workgroups start; which workgroup computes a
    split changes none of its partials, so out and lse equal the static order
    (NULL counters) bit for bit, call after call, and the ticket is back at zero
    after every call (also after a smaller batch on the same counters)."""
    from llm_cuda import _native

    g = torch.Generator().manual_seed(B + split)
    lens = torch.randint(lo, hi + 1, (B,), generator=g).tolist()
    Hq, Hkv, D, P = 32, 8, 128, 64
    q, kp, vp, bt, sl = _paged_case(lens, Hq, Hkv, D, P, torch.bfloat16, cuda, seed=B,
                                    poison=False)
    q, kp, vp, bt, sl = (t.to(cuda) for t in (q, kp, vp, bt, sl))
    counters = torch.zeros(_native.load().lc_paged_decode_counter_count(), dtype=torch.int32,
                           device=cuda)
    ref_out, ref_lse = _abi_decode(q, kp, vp, bt, sl, split, None)
    for call in range(3):
        out, lse = _abi_decode(q, kp, vp, bt, sl, split, counters)
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), f"call {call}: output differs from the static order"
        assert torch.equal(lse, ref_lse), f"call {call}: lse differs from the static order"
        assert int(counters.abs().sum()) == 0, f"call {call}: ticket not returned to zero"
    half = B // 2
    out_h, lse_h = _abi_decode(q[:half], kp, vp, bt[:half], sl[:half], split, counters)
    ref_h, ref_lse_h = _abi_decode(q[:half], kp, vp, bt[:half], sl[:half], split, None)
    torch.cuda.synchronize()
    assert torch.equal(out_h, ref_h) and torch.equal(lse_h, ref_lse_h)
    assert int(counters.abs().sum()) == 0
    ref, ref_l = paged_decode(q.cpu(), kp.cpu(), vp.cpu(), bt.cpu(), sl.cpu())
    assert_close(ref_out, ref, ATOL[torch.bfloat16], f"B={B} vs oracle")
    assert_lse_close(ref_lse, ref_l)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_running_max_rescales(cuda, dtype):
    """Keys whose scores jump by ~8.7 log2 units every 64 tokens: the lazy
    rescale of O and l (a running max growing by more than 2^8) runs once per
    64 tokens inside every split, which N(0,1) inputs never trigger past the
    first step."""
    lens = [130, 700, 1025, 64]
    Hq, Hkv, D, P = 8, 2, 128, 64
    q, kp, vp, bt, sl = _paged_case(lens, Hq, Hkv, D, P, dtype, cuda, seed=17, poison=False)
    g = torch.Generator().manual_seed(18)
    unit = D ** 0.5
    for b, L in enumerate(lens):
        for t0 in range(0, L, P):
            page = int(bt[b, t0 // P])
            pos = torch.arange(t0, t0 + P)
            t = 6.0 * (pos // 64).float() / unit
            kp[page] = (t[None, :, None] * torch.ones(Hkv, P, D)
                        + 0.3 * torch.randn(Hkv, P, D, generator=g)).to(dtype)
    q = (torch.ones(len(lens), Hq, 1, D) + 0.1 * torch.randn(len(lens), Hq, 1, D, generator=g)).to(dtype)
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert ref_lse.max().item() > 3 * 6.0
    assert_close(out, ref, ATOL[dtype], "paged rescales")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_paged_lengths_outside_the_table_are_clamped(cuda, dtype):
    """seq_lens past the block table's capacity read only the table's tokens;
    a negative length reads none (zeros, lse -inf). Nothing past the table is
    dereferenced (the pools' free slots are NaN)."""
    lens = [130, 64, 200]
    q, kp, vp, bt, sl = _paged_case(lens, 8, 2, 128, 64, dtype, cuda, seed=21, poison=False,
                                    extra_pages=0)
    cap = bt.shape[1] * 64
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    # rows 0 and 2 read every token of the pages their table row holds (the row is
    # padded with -1 past the sequence's pages, and those entries drop out)
    sl_bad = torch.tensor([cap + 1000, 64, 1 << 30], dtype=torch.int32)
    out, lse = _run_paged(q, kp, vp, bt, sl_bad, cuda)
    assert_close(out[1:2], ref[1:2], ATOL[dtype], "in-range row")
    assert_lse_close(lse[1:2], ref_lse[1:2])
    for b in (0, 2):
        own = int((bt[b] >= 0).sum())
        kk = torch.cat([kp[int(bt[b, i])] for i in range(own)], dim=1)[None]
        vv = torch.cat([vp[int(bt[b, i])] for i in range(own)], dim=1)[None]
        r, rl = decode_attention(q[b:b + 1], kk, vv)
        assert_close(out[b:b + 1], r, ATOL[dtype], f"clamped row {b}")
        assert_lse_close(lse[b:b + 1], rl)
    out, lse = _run_paged(q, kp, vp, bt, torch.tensor([-7, 64, 0], dtype=torch.int32), cuda)
    assert (out[0].float().cpu() == 0).all() and torch.isinf(lse[0].cpu()).all()
    assert (out[2].float().cpu() == 0).all() and torch.isinf(lse[2].cpu()).all()


def test_unaligned_split_touching_65_pages(cuda):
    """Page size 160 with 10176-token splits: the second split starts 96 tokens
    into a page and touches 65 pages, one more than the row kernel's
    one-page-per-lane table holds; such a launch must take a kernel that
    resolves every page (the first split touches 64)."""
    lens = [20500, 10300]
    q, kp, vp, bt, sl = _paged_case(lens, 8, 2, 128, 160, torch.bfloat16, cuda, seed=31)
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda, split_tokens=10176)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert_close(out, ref, ATOL[torch.bfloat16], "65-page split")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 48])
@pytest.mark.parametrize("P", [16, 48])
def test_paged_lanes_kernel_small_head_dim(cuda, dtype, D, P):
    """Page sizes that are not multiples of 32 run the per-lane-page kernel; at
    head_dim <= 64 it is the 64-wide instance (48 is padded to 64)."""
    lens = [1, 17, 96, 200, 511, 47]
    q, kp, vp, bt, sl = _paged_case(lens, 16, 4, D, P, dtype, cuda, seed=D + P)
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert_close(out, ref, ATOL[dtype], f"lanes D={D} P={P}")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Hq,Hkv,D,P", [(32, 8, 128, 64), (16, 4, 64, 32), (8, 2, 256, 128),
                                        (40, 2, 48, 64), (8, 1, 128, 96)])
def test_single_split_workgroup_kernel(cuda, dtype, Hq, Hkv, D, P):
    """One split covering the capacity (max_splits == 1) runs one workgroup of
    several waves per (sequence, group of <= 16 query heads): the steps are
    dealt out to the waves by the device-side length and the waves' softmax
    states merge in LDS, with no merge kernel. Lengths 0, 1, fewer steps than
    waves, one token past a step, ragged, and a full 2049-token context; G = 20
    spans two head groups; head_dim 48 is padded to 64."""
    lens = [0, 1, 31, 33, 257, 1000, 2049]
    q, kp, vp, bt, sl = _paged_case(lens, Hq, Hkv, D, P, dtype, cuda, seed=Hq + D + P)
    split = -(-bt.shape[1] * P // 64) * 64
    out, lse = _run_paged(q, kp, vp, bt, sl, cuda, split_tokens=split)
    ref, ref_lse = paged_decode(q, kp, vp, bt, sl)
    assert (out[0].float().cpu() == 0).all() and torch.isinf(lse[0].cpu()).all()
    assert_close(out[1:], ref[1:], ATOL[dtype], f"single split Hq={Hq} D={D} P={P}")
    assert_lse_close(lse[1:], ref_lse[1:])
    # the split-K path on the same inputs agrees to fp32 rounding of the merge
    out2, lse2 = _run_paged(q, kp, vp, bt, sl, cuda, split_tokens=256)
    assert_close(out, out2, ATOL[dtype], "single split vs split-K")
    assert_lse_close(lse, lse2)


def test_single_split_invalid_entry_and_clamped_length(cuda):
    """Single-split kernel: a bad page id inside the live range drops that
    page's tokens, and lengths beyond the table capacity are clamped to it."""
    lens = [192, 100]
    q, kp, vp, bt, sl = _paged_case(lens, 16, 2, 128, 64, torch.bfloat16, cuda, seed=41,
                                    poison=False)
    good = bt.clone()
    bt[0, 1] = -5
    sl_run = torch.tensor([192, 10 ** 6], dtype=torch.int32)  # 1e6 clamps to 192
    out, lse = _run_paged(q, kp, vp, bt, sl_run, cuda, split_tokens=192)
    keep = [0, 2]
    kk = torch.cat([kp[int(good[0, i])] for i in keep], dim=1)[None]
    vv = torch.cat([vp[int(good[0, i])] for i in keep], dim=1)[None]
    ref0, ref0_lse = decode_attention(q[:1], kk, vv)
    assert_close(out[:1], ref0, ATOL[torch.bfloat16], "single split, invalid page")
    assert_lse_close(lse[:1], ref0_lse)
    # sequence 1 owns two pages; its third entry is -1, so of the clamped 192
    # tokens the first 128 remain
    kk = torch.cat([kp[int(bt[1, i])] for i in (0, 1)], dim=1)[None]
    vv = torch.cat([vp[int(bt[1, i])] for i in (0, 1)], dim=1)[None]
    ref1, ref1_lse = decode_attention(q[1:], kk, vv)
    assert_close(out[1:], ref1, ATOL[torch.bfloat16], "single split, clamped length")
    assert_lse_close(lse[1:], ref1_lse)

