"""Flash-decode entries (reference: kernels/triton/decode_attention.py:162-287).

* `triton_decode_attention(q, k, v)` keeps the reference signature: one query
  token against contiguous per-sequence K/V [B, Hkv, L, D]. It runs the same
  split-K kernel as the paged entry, describing each sequence's K/V as a
  single page of L tokens.
* `paged_decode_attention(q, key_pages, value_pages, block_table, seq_lens)`
  is the entry the model uses: K/V are read in place from the page pools
  [N, Hkv, P, D] through an int32 block table [B, max_pages] with ragged
  int32 seq_lens [B] (the reference could only decode a contiguous copy of a
  batch-1 cache, models/llama3/kv_cache.py:43-44,65-83).

Both return out shaped like q; `return_lse=True` adds the fp32 natural-log
logsumexp [B, Hq] of the scaled scores. The paged entry also takes the
reference's additive attention_mask (the reference's decode predicate refuses
masks and falls back to torch; that predicate keeps its answer here).
"""
from __future__ import annotations

import torch

from llm_cuda.kernels import _ops

_MAX_HEAD_DIM = 256

_TABLE_CACHE: dict = {}


def can_use_triton_decode_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    attention_mask: torch.Tensor | None = None,
) -> bool:
    """Same guards as the reference predicate (decode_attention.py:162-201)."""
    if attention_mask is not None:
        return False
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return False
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        return False
    if q.shape[-2] != 1:
        return False
    if q.shape[0] != k.shape[0] or q.shape[0] != v.shape[0]:
        return False
    if q.shape[-1] != k.shape[-1] or q.shape[-1] != v.shape[-1]:
        return False
    if q.shape[-1] > _MAX_HEAD_DIM:
        return False
    if k.shape != v.shape:
        return False
    if k.shape[-2] == 0:
        return False
    n_heads, n_kv_heads = q.shape[1], k.shape[1]
    if n_kv_heads == 0 or n_heads % n_kv_heads != 0:
        return False
    if not (q.dtype == k.dtype == v.dtype):
        return False
    return True


def _identity_table(batch: int, length: int, device: torch.device):
    key = (batch, length, device)
    hit = _TABLE_CACHE.get(key)
    if hit is None:
        if len(_TABLE_CACHE) > 64:
            _TABLE_CACHE.clear()
        table = torch.arange(batch, dtype=torch.int32, device=device).view(batch, 1)
        lens = torch.full((batch,), length, dtype=torch.int32, device=device)
        hit = (table, lens)
        _TABLE_CACHE[key] = hit
    return hit


def triton_decode_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    return_lse: bool = False,
):
    """q [B, Hq, 1, D]; k, v [B, Hkv, L, D] (any strides with unit head_dim stride)."""
    if q.dim() != 4 or q.shape[-2] != 1 or k.dim() != 4 or k.shape != v.shape:
        raise ValueError("expected q [B, Hq, 1, D] and k, v [B, Hkv, L, D]")
    if k.stride() != v.stride() or k.stride(-1) != 1:
        k = k.contiguous()
        v = v.contiguous()
    B, Hkv, L, D = k.shape
    if L == 0:
        raise ValueError("kv_len must be > 0")
    # Each sequence is one page of L tokens: page b starts at b * k.stride(0).
    pages_k = k.as_strided((B, Hkv, L, D), k.stride())
    pages_v = v.as_strided((B, Hkv, L, D), v.stride())
    table, lens = _identity_table(B, L, q.device)
    return _ops.paged_decode(q, pages_k, pages_v, table, lens, return_lse=return_lse,
                             uniform_length=L)


def paged_decode_attention(
    q: torch.Tensor,
    key_pages: torch.Tensor,
    value_pages: torch.Tensor,
    block_table: torch.Tensor,
    seq_lens: torch.Tensor,
    scale: float | None = None,
    return_lse: bool = False,
    split_tokens: int | None = None,
    workspace: torch.Tensor | None = None,
    attention_mask: torch.Tensor | None = None,
    uniform_length: int | None = None,
):
    """attention_mask: the reference's additive mask for the query token,
    broadcastable to [B, Hq, 1, L]; token t < L of each sequence gets
    mask[..., t] added to its scaled score (models/llama3/attention.py:85-86),
    later tokens none. uniform_length: every seq_lens entry is known to equal
    this (a split-choice hint; the result does not depend on it)."""
    return _ops.paged_decode(q, key_pages, value_pages, block_table, seq_lens, scale=scale,
                             return_lse=return_lse, split_tokens=split_tokens,
                             workspace=workspace, attention_mask=attention_mask,
                             uniform_length=uniform_length)
