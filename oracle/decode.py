"""Decode-attention and paged-KV oracle. TEST INFRASTRUCTURE ONLY.

decode_attention follows the reference's test oracle
tests/test_triton_decode_attention.py:26-58 (per (b, h): kv head h // G,
scores = k @ q * scale, softmax, probs-weighted sum of v), in fp32, returning
also the natural-log logsumexp.

gather_pages restates the page addressing of models/llama3/kv_cache.py:55-61
(token t -> page t // P, slot t % P) with the identity page mapping replaced
by a block table, in numpy integer arithmetic (bit-exact by construction: it
only copies elements).
"""
from __future__ import annotations

import math

import numpy as np
import torch


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     scale: float | None = None, bias: torch.Tensor | None = None):
    """q [B, Hq, 1, D]; k, v [B, Hkv, L, D] -> (o fp32 [B, Hq, 1, D], lse fp32 [B, Hq]).

    bias: the reference's additive attention_mask for the query token,
    broadcastable to [B, Hq, L] (models/llama3/attention.py:85-86 adds it to
    the scaled scores before the softmax). Rows without a finite score give
    o = 0, lse = -inf.
    """
    from .attention import _softmax_rows

    B, Hq, _, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    bv = None if bias is None else torch.broadcast_to(bias.float(), (B, Hq, L))
    out = torch.empty((B, Hq, 1, D), dtype=torch.float32)
    lse = torch.empty((B, Hq), dtype=torch.float32)
    for b in range(B):
        for kvh in range(Hkv):
            hs = slice(kvh * G, (kvh + 1) * G)
            qg = q[b, hs, 0, :].float()                      # [G, D]
            kk = k[b, kvh].float()                           # [L, D]
            vv = v[b, kvh].float()
            s = torch.matmul(qg, kk.t()) * scale             # [G, L]
            if bv is not None:
                s = s + bv[b, hs]
            p, row_lse = _softmax_rows(s)
            out[b, hs, 0, :] = torch.matmul(p, vv)
            lse[b, hs] = row_lse
    return out, lse


def gather_pages(pages: np.ndarray, block_table: np.ndarray, length: int) -> np.ndarray:
    """pages [N, H, P, D]; block_table int [B, max_pages] -> [B, H, length, D].

    out[b, :, t, :] = pages[block_table[b, t // P], :, t % P, :].
    """
    pages = np.asarray(pages)
    bt = np.asarray(block_table).astype(np.int64)
    P = pages.shape[2]
    t = np.arange(length, dtype=np.int64)
    page_idx = t // P
    slot = t % P
    phys = bt[:, page_idx]                               # [B, length]
    g = pages[phys, :, slot[None, :], :]                 # [B, length, H, D]
    return np.ascontiguousarray(np.transpose(g, (0, 2, 1, 3)))


def gather_pages_torch(pages: torch.Tensor, block_table: torch.Tensor, length: int) -> torch.Tensor:
    """gather_pages for host torch tensors of any dtype (via a raw int view)."""
    raw = pages.contiguous().view(torch.int16 if pages.element_size() == 2 else torch.int32)
    g = gather_pages(raw.numpy(), block_table.cpu().numpy(), length)
    return torch.from_numpy(g).view(pages.dtype)


def paged_decode(q: torch.Tensor, key_pages: torch.Tensor, value_pages: torch.Tensor,
                 block_table: torch.Tensor, seq_lens, scale: float | None = None,
                 bias: torch.Tensor | None = None):
    """Per-sequence gather through the block table, then decode_attention.

    Empty sequences give o = 0, lse = -inf (the kernel's documented behaviour).
    bias: [B, Hq or 1, Lb] additive scores of token t < Lb of each sequence
    (tokens at or past Lb get none).
    """
    B, Hq, _, D = q.shape
    out = torch.zeros((B, Hq, 1, D), dtype=torch.float32)
    lse = torch.full((B, Hq), float("-inf"), dtype=torch.float32)
    lens = [int(x) for x in (seq_lens.tolist() if torch.is_tensor(seq_lens) else seq_lens)]
    bt = block_table.cpu()
    for b in range(B):
        L = lens[b]
        if L <= 0:
            continue
        kk = gather_pages_torch(key_pages, bt[b:b + 1], L)
        vv = gather_pages_torch(value_pages, bt[b:b + 1], L)
        bb = None
        if bias is not None:
            row = bias[b:b + 1].float()
            bb = torch.zeros(1, row.shape[1], L)
            n = min(L, row.shape[-1])
            bb[..., :n] = row[..., :n]
        o, l_ = decode_attention(q[b:b + 1], kk, vv, scale, bias=bb)
        out[b] = o[0]
        lse[b] = l_[0]
    return out, lse


def merge_splits(part_o: torch.Tensor, part_lse: torch.Tensor):
    """Combine per-split normalised outputs [S, ..., D] and lses [S, ...].

    lse = logsumexp_s(lse_s); o = sum_s exp(lse_s - lse) * o_s.
    """
    lse = torch.logsumexp(part_lse, dim=0)
    w = torch.exp(part_lse - lse.unsqueeze(0))
    return (w.unsqueeze(-1) * part_o).sum(dim=0), lse
