"""C-ABI boundary and host-side checks that need no GPU.

The library must load, export exactly the entry points include/lcuda.h
declares, and reject bad arguments before any launch (negative status plus a
message). The Python entry points must reject host tensors instead of
computing on the CPU, and keep the reference's predicate/None contracts
(kernels/cuda/*.py, kernels/triton/*_attention.py, rope.py).
"""
import ctypes
import re

import pytest
import torch

from conftest import ROOT

HEADER = ROOT / "include" / "lcuda.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"LC_API\s+[\w\s\*]+?\b(lc_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "lc_paged_decode_fwd" in names and "lc_prefill_attn_fwd" in names
    assert len(names) >= 10


def test_library_exports_every_declared_symbol():
    from llm_cuda import _native

    lib = _native.load()
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in lcuda.h but not exported"
    assert set(_declared()) == set(_native.EXPORTS), "ctypes signatures out of sync with lcuda.h"
    assert lib.lc_version() >= 100


def test_exports_nothing_else():
    import subprocess

    from llm_cuda import _native

    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = sorted({ln.split()[-1] for ln in out.splitlines() if " T " in ln})
    assert exported == _declared()


def test_decode_linear_arguments_rejected_before_launch():
    from llm_cuda import _native

    lib = _native.load()
    # one counter per row block of the smaller shape (64 rows; 32 output
    # columns in mode 1)
    assert lib.lc_decode_linear_counter_count(4096, 0) == 64
    assert lib.lc_decode_linear_counter_count(14336, 1) == 448
    assert lib.lc_decode_linear_workspace_bytes(32, 4096, 4096, 2, 0) == -1
    # one workgroup per row block: no partials
    assert lib.lc_decode_linear_workspace_bytes(32, 4096, 4096, 0, 1) == 256
    # K % 256 == 0: 64-row blocks of 16 tiles, 8 workgroups each; two fp32
    # partials of 64 x 32 values per workgroup (its first and last block)
    assert lib.lc_decode_linear_workspace_bytes(32, 4096, 4096, 0, 8) == 64 * 8 * 2 * 2048 * 4
    # K % 256 == 128: 128-row blocks of 33 tiles, 3 workgroups each
    assert lib.lc_decode_linear_workspace_bytes(32, 4096, 4224, 0, 3) == 32 * 3 * 2 * 4096 * 4
    # the library's grid with 512 one-tile blocks: runs of two whole blocks,
    # no partials (256 CUs where no GPU is visible)
    assert lib.lc_decode_linear_workspace_bytes(1, 32768, 256, 0, 0) == 256
    for M, K, mode, what in ((33, 512, 0, b"M=33"), (4, 500, 0, b"multiple of 128"),
                             (4, 512, 3, b"mode 3")):
        rc = lib.lc_decode_linear(16, K, 16, K, 16, 256, M, 256, K, mode, 0, 16, 1 << 20, 16, 2,
                                  None)
        assert rc == -1 and what in lib.lc_last_error(), lib.lc_last_error()
    rc = lib.lc_decode_linear(16, 512, 16, 512, 16, 256, 4, 256, 512, 0, 0, 16, 1 << 20, 16, 0,
                              None)
    assert rc == -1 and b"dtype" in lib.lc_last_error()


def test_invalid_arguments_rejected_before_launch():
    from llm_cuda import _native

    lib = _native.load()
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    # null pointers
    rc = lib.lc_rmsnorm_fwd(None, None, None, 4, 8, 8, 8, 1e-5, 2, 2, None)
    assert rc == -1 and b"null" in lib.lc_last_error()
    # Hq not a multiple of Hkv
    rc = lib.lc_prefill_attn_fwd(8, 8, 8, 8, None, 1, 5, 3, 4, 4, 16, st, st, st, st, 0, None,
                                 None, 0, None, 1.0, 2, None)
    assert rc == -1 and b"multiple" in lib.lc_last_error()
    # a bias without strides, or of a third dtype
    rc = lib.lc_prefill_attn_fwd(8, 8, 8, 8, None, 1, 4, 2, 4, 4, 16, st, st, st, st, 0, 8,
                                 None, 0, None, 1.0, 2, None)
    assert rc == -1 and b"bias_strides" in lib.lc_last_error()
    rc = lib.lc_prefill_attn_fwd(8, 8, 8, 8, None, 1, 4, 2, 4, 4, 16, st, st, st, st, 0, 8,
                                 st, 1, None, 1.0, 2, None)
    assert rc == -1 and b"bias dtype" in lib.lc_last_error()
    # odd head_dim for RoPE
    rc = lib.lc_rope_fwd(8, 8, 1, st, st, None, None, 0, None, None, 8, 8, 15, 15, 1, 1, 15, 2,
                         None)
    assert rc == -1 and b"even" in lib.lc_last_error()
    # split does not cover the table capacity
    rc = lib.lc_paged_decode_fwd(8, 128, 128, 8, 8, 1, 1, 1, 8, 4, 4, 16, 8, 8, 128, 128, None,
                                 None, 0, 0, 0, 0, 256, 1 << 20, None, 1, 4, 2, 128, 64, 64, 1,
                                 1.0, 2, None)
    assert rc == -1 and b"capacity" in lib.lc_last_error()
    # workspace too small
    rc = lib.lc_paged_decode_fwd(8, 128, 128, 8, 8, 1, 1, 1, 8, 4, 4, 16, 8, 8, 128, 128, None,
                                 None, 0, 0, 0, 0, 256, 16, None, 1, 4, 2, 128, 64, 64, 4, 1.0,
                                 2, None)
    assert rc == -1 and b"workspace" in lib.lc_last_error()
    # negative bias stride
    rc = lib.lc_paged_decode_fwd(8, 128, 128, 8, 8, 1, 1, 1, 8, 4, 4, 16, 8, 8, 128, 128, None,
                                 8, -1, 0, 16, 0, 256, 1 << 20, None, 1, 4, 2, 128, 64, 64, 4,
                                 1.0, 2, None)
    assert rc == -1 and b"bias" in lib.lc_last_error()
    # unknown dtype
    rc = lib.lc_swiglu_fwd(8, 8, 8, 2, 8, 8, 8, 8, 7, None)
    assert rc == -1 and b"dtype" in lib.lc_last_error()


def test_workspace_size_formula():
    from llm_cuda import _native

    lib = _native.load()
    n = 2 * 4 * 3
    expect = ((n * 128 * 4 + 255) // 256) * 256 + n * 4
    assert lib.lc_paged_decode_workspace_bytes(2, 4, 128, 3) == expect
    assert lib.lc_paged_decode_workspace_bytes(-1, 4, 128, 3) == -1


def test_host_tensors_rejected():
    from llm_cuda.kernels.triton.attention import triton_fused_causal_attention
    from llm_cuda.kernels.triton.decode_attention import triton_decode_attention
    from llm_cuda.kernels.triton.rmsnorm import triton_rms_norm
    from llm_cuda.kernels.triton.rope import triton_apply_rope
    from llm_cuda.kernels.triton.swiglu import triton_swiglu

    x = torch.randn(2, 4, 16)
    with pytest.raises(RuntimeError, match="ROCm"):
        triton_rms_norm(x, torch.ones(16), 1e-5)
    with pytest.raises(RuntimeError, match="ROCm"):
        triton_swiglu(x, x)
    q = torch.randn(1, 2, 8, 16)
    with pytest.raises(RuntimeError, match="ROCm"):
        triton_fused_causal_attention(q, q, q)
    with pytest.raises(RuntimeError, match="ROCm"):
        triton_apply_rope(q, torch.randn(8, 16), torch.randn(8, 16))
    with pytest.raises(RuntimeError, match="ROCm"):
        triton_decode_attention(torch.randn(1, 2, 1, 16), q, q)


def test_reference_none_contracts_on_host():
    """kernels/cuda/*.py return None for host tensors (reference test_cuda_extension.py:21-53)."""
    from llm_cuda.kernels.cuda.attention import cuda_causal_attention_extension
    from llm_cuda.kernels.cuda.rmsnorm import cuda_extension_status, cuda_rms_norm_extension
    from llm_cuda.kernels.cuda.swiglu import cuda_swiglu_extension

    x = torch.randn(2, 4, 16)
    assert cuda_rms_norm_extension(x, torch.randn(16), 1e-5) is None
    assert cuda_swiglu_extension(x, torch.randn_like(x)) is None
    q = torch.randn(1, 2, 8, 16)
    assert cuda_causal_attention_extension(q, q, q) is None
    status = cuda_extension_status()
    assert isinstance(status, str) and status


def test_predicates_false_on_host():
    """Guards keep the reference's answers for host tensors and bad shapes
    (test_triton_decode_attention.py:66-136, test_triton_rope.py:46-93)."""
    from llm_cuda.kernels.triton.attention import can_use_triton_fused_attention
    from llm_cuda.kernels.triton.decode_attention import can_use_triton_decode_attention
    from llm_cuda.kernels.triton.rope import can_use_triton_rope

    q = torch.randn(1, 4, 1, 16, dtype=torch.float16)
    k = torch.randn(1, 2, 8, 16, dtype=torch.float16)
    assert can_use_triton_decode_attention(q, k, k) is False
    assert can_use_triton_fused_attention(q, k, k) is False
    x = torch.randn(1, 4, 4, 16)
    assert can_use_triton_rope(x, torch.randn(4, 16), torch.randn(4, 16)) is False


def test_config_validation():
    from llm_cuda.models.llama3.config import Llama3Config

    cfg = Llama3Config(hidden_size=256, num_attention_heads=8, num_key_value_heads=2)
    assert cfg.head_dim == 32
    with pytest.raises(ValueError):
        Llama3Config(hidden_size=250, num_attention_heads=8)
    with pytest.raises(ValueError):
        Llama3Config(tensor_parallel_size=0)
    with pytest.raises(ValueError):
        Llama3Config(hidden_size=256, num_attention_heads=8, num_key_value_heads=3)


def test_kv_cache_argument_checks():
    from llm_cuda.models.llama3.kv_cache import PagedKVLayerCache

    with pytest.raises(ValueError):
        PagedKVLayerCache(2, 8, 16, 0, torch.device("cpu"), torch.float32)
    with pytest.raises(ValueError):
        PagedKVLayerCache(2, 8, 0, 4, torch.device("cpu"), torch.float32)
    c = PagedKVLayerCache(2, 8, 10, 4, torch.device("cpu"), torch.float32, batch_size=3)
    assert c.max_pages == 3 and c.block_table.shape == (3, 3)
    assert c.block_table.flatten().tolist() == list(range(9))
    assert c.length == 0
    with pytest.raises(ValueError, match="batch"):
        c.append(torch.zeros(1, 2, 1, 8), torch.zeros(1, 2, 1, 8))
    with pytest.raises(ValueError, match="max_seq_len"):
        c.append(torch.zeros(3, 2, 11, 8), torch.zeros(3, 2, 11, 8))


def test_split_heuristic():
    from llm_cuda.kernels._ops import choose_split_tokens, takes_workgroup_splits

    # config 2 (64 ragged sequences, 512 units, capacity 8000): three
    # workgroup splits per unit, 8000 / 3 rounded up to 3072 tokens
    assert choose_split_tokens(64, 8, 4, 8000) == 3072
    assert takes_workgroup_splits(512, 3072, 3, 64, 128, 8000)
    # more than 256 sequences (no longest-first order): about 8 splits per CU,
    # here one per unit (2056 units)
    assert choose_split_tokens(257, 8, 4, 8000) == 8000
    # config 4 (32 sequences at 2049 tokens, 256 units): one split over the
    # capacity when the common length is known; when not, six splits per unit
    # would be 352 tokens, so the 2048-token floor; over 256 sequences with
    # fewer units than 8 rounds of the CUs, 512-token one-wave splits
    assert choose_split_tokens(32, 8, 4, 2112, 64, 128, 2049) == 2112
    assert choose_split_tokens(32, 8, 4, 2112) == 2048
    assert choose_split_tokens(257, 1, 4, 2112) == 512
    assert not takes_workgroup_splits(257, 512, 5, 64, 128, 2112)
    # long ragged contexts: more splits until a wave's share fits 64 pages
    # (100000 / 3 -> 34816 would give 68 pages per wave; 100000 / 4 -> 25600)
    assert choose_split_tokens(64, 8, 4, 100000) == 25600
    assert takes_workgroup_splits(512, 25600, 4, 64, 128, 100000)
    # config 5 (8 sequences of 32K tokens, 64 units): 4 splits per unit, one
    # round of the CUs, known length or not
    assert choose_split_tokens(8, 8, 8, 32768) == 8192
    assert choose_split_tokens(8, 8, 8, 32768, 64, 128, 32768) == 8192
    # one sequence of 32K tokens (8 units): 32 splits, small grid -> workgroups
    assert choose_split_tokens(1, 8, 4, 32832) == 1088
    assert takes_workgroup_splits(8, 1088, 31, 64, 128, 32832)
    # equal lengths: the fewest splits per unit that fill rounds of the CUs
    assert choose_split_tokens(64, 8, 4, 4160, 64, 128, 4096) == 4160  # 512 units, 1 split
    assert choose_split_tokens(48, 8, 4, 8192, 64, 128, 8000) == 4032  # 384 units, 2 splits
    # an empty batch launches nothing: any multiple of 64 covering the capacity
    assert choose_split_tokens(0, 8, 4, 8000) == 8000
    assert choose_split_tokens(0, 8, 4, 8000, 64, 128, 100) == 8000
    # pages of 48 tokens: one-wave splits only
    assert choose_split_tokens(64, 8, 4, 8000, 48) == 512
    assert choose_split_tokens(1, 2, 4, 128, 48) == 64
    for args in [(1, 1, 1, 1), (3, 5, 7, 1000), (64, 8, 16, 100000), (2, 8, 8, 65536)]:
        s = choose_split_tokens(*args)
        assert s % 64 == 0 and s >= 64


def test_single_split_fit_matches_the_library_rule():
    """single_split_fits mirrors the C dispatch rule: 8 waves up to head_dim
    128 (4 above), each wave's whole 32-token steps within 64 pages."""
    from llm_cuda.kernels._ops import single_split_fits

    # a wave's range starts on a 32-token step, so 4032 tokens (126 steps)
    # touch at most 64 pages of 64: 8 x 4032 = 32256 tokens is the largest
    # capacity, 4 x 4032 = 16128 at head_dim 256
    assert single_split_fits(32256, 64, 128)
    assert not single_split_fits(32257, 64, 128)
    assert single_split_fits(16128, 64, 256) and not single_split_fits(16129, 64, 256)
    assert not single_split_fits(1024, 48, 128)


def test_reference_attention_selectors_are_importable():
    """test_triton_attention.py:50-76 of the reference, on this package: the
    tiling helpers keep the reference's policy; SDPA is never selected."""
    import torch

    from llm_cuda.kernels.triton.attention import (
        _select_attention_block_sizes,
        _select_attention_num_warps,
        _cuda_sdpa_causal_attention,
        _should_use_cuda_sdpa,
        can_use_triton_fused_attention,
    )

    assert _select_attention_block_sizes(seq_len=128, head_dim=64) == (32, 64)
    assert _select_attention_block_sizes(seq_len=512, head_dim=64) == (64, 64)
    assert _select_attention_block_sizes(seq_len=2048, head_dim=64) == (128, 64)
    assert _select_attention_block_sizes(seq_len=8, head_dim=5) == (32, 16)
    assert _select_attention_block_sizes(seq_len=8, head_dim=256) == (32, 128)
    assert _select_attention_num_warps(64, 128) == 8
    assert _select_attention_num_warps(64, 64) == 4
    assert _select_attention_num_warps(16, 32) == 2
    q = torch.randn(1, 2, 1024, 64, dtype=torch.float16)
    assert _should_use_cuda_sdpa(q, q, q, attention_mask=None) is False
    assert can_use_triton_fused_attention(q[:, :, :8, :32], q[:, :, :8, :32], q[:, :, :8, :32]) is False
    # the reference's SDPA helper keeps its name but runs the HIP kernel: on host
    # tensors it raises rather than computing anything on the CPU
    with pytest.raises((RuntimeError, ValueError)):
        _cuda_sdpa_causal_attention(q, q, q)


def test_empty_extents_accept_null_pointers():
    """Empty tensors may carry null data pointers: an empty query set is a no-op,
    a null pointer behind a non-empty extent is rejected before any launch."""
    from llm_cuda import _native

    lib = _native.load()
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    rc = lib.lc_prefill_attn_fwd(None, 8, 8, None, None, 1, 4, 2, 0, 16, 64, st, st, st, st, 0,
                                 None, None, 0, None, 1.0, 2, None)
    assert rc == 0
    rc = lib.lc_prefill_attn_fwd(None, 8, 8, 8, None, 1, 4, 2, 3, 16, 64, st, st, st, st, 0, None,
                                 None, 0, None, 1.0, 2, None)
    assert rc == -1 and b"null q" in lib.lc_last_error()
    rc = lib.lc_prefill_attn_fwd(8, None, 8, 8, None, 1, 4, 2, 3, 16, 64, st, st, st, st, 0, None,
                                 None, 0, None, 1.0, 2, None)
    assert rc == -1 and b"null k" in lib.lc_last_error()


def test_every_entry_accepts_empty_work_with_null_pointers():
    """Zero rows / tokens / batch: LC_OK without a launch, whatever the pointers."""
    from llm_cuda import _native

    lib = _native.load()
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    assert lib.lc_rmsnorm_fwd(None, None, None, 0, 8, 8, 8, 1e-5, 2, 2, None) == 0
    assert lib.lc_add_rmsnorm_fwd(None, None, None, None, None, 0, 8, 8, 8, 8, 8, 1e-5, 2, 2,
                                  None) == 0
    assert lib.lc_swiglu_fwd(None, None, None, 0, 8, 8, 8, 8, 2, None) == 0
    assert lib.lc_rope_fwd(None, None, 1, st, st, None, None, 0, None, None, None, None, 8, 8, 0,
                           4, 8, 2, None) == 0
    assert lib.lc_lm_head_argmax(None, 8, None, 8, 0, 8, 8, None, None, None, 0, None, 2,
                                 None) == 0
    assert lib.lc_prefill_attn_bwd(None, None, None, None, None, None, None, None, None, 0, 4, 2,
                                   8, 8, 64, st, st, st, st, st, st, st, st, 0, None, None, 0, 1.0,
                                   None, 0, 2, None) == 0
    # a null pointer behind real work is still an error
    assert lib.lc_swiglu_fwd(None, None, None, 2, 8, 8, 8, 8, 2, None) == -1
    assert lib.lc_lm_head_argmax(None, 8, None, 8, 2, 8, 8, None, None, None, 4096, None, 2,
                                 None) == -1


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """No silent fallback: without the built library every kernel call raises."""
    import pytest

    from llm_cuda import _native

    monkeypatch.setattr(_native, "_LIB", None)
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "missing" / "liblcuda_hip.so")
    with pytest.raises(_native.NativeError):
        _native.load()
    assert _native.status().startswith("failed")
