"""Causal attention oracle (fp32 on the host). TEST INFRASTRUCTURE ONLY.

Follows the reference's torch fallback kernels/triton/attention.py:457-477
(scores = q k^T * scale, triu(-inf, 1) causal mask, `+ attention_mask`,
softmax, probs @ v) and, for a cached prefix, models/llama3/attention.py:63-89
(key j visible to query i iff j <= past_len + i, then `+ attention_mask`).
GQA is expressed as the reference's repeat-KV (models/llama3/attention.py:
56-61): query head h reads kv head h // G. Returns the output and the
natural-log logsumexp of the masked scores.

`bias` is the reference's additive attention_mask, broadcastable to
[B, Hq, Sq, Skv] and added to the scaled scores in fp32. The softmax is the
reference's (torch.softmax: exp(s - rowmax) / sum), so a row whose visible
scores are all equal (e.g. all pushed to the same huge negative value by a
finfo.min mask) averages them uniformly. A row with no finite score (no
visible key, or every visible key at -inf) gives o = 0 and lse = -inf; the
reference's torch path gives NaN there.
"""
from __future__ import annotations

import math

import torch


def _bias_view(bias, B, Hq, Sq, Skv):
    if bias is None:
        return None
    return torch.broadcast_to(bias.float(), (B, Hq, Sq, Skv))


def _softmax_rows(s: torch.Tensor):
    """(p, lse) of rows of s; rows without a finite entry give p = 0, lse = -inf."""
    if s.shape[-1] == 0:
        return torch.zeros_like(s), torch.full(s.shape[:-1], float("-inf"))
    m = s.amax(dim=-1, keepdim=True)
    ok = torch.isfinite(m)
    m0 = torch.where(ok, m, torch.zeros_like(m))
    e = torch.exp(s - m0)
    e = torch.where(ok, e, torch.zeros_like(e))
    z = e.sum(dim=-1, keepdim=True)
    p = e / torch.where(ok, z, torch.ones_like(z))
    lse = torch.where(ok, m0 + torch.log(z), torch.full_like(m, float("-inf")))
    return p, lse.squeeze(-1)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_offset: int = 0,
                     scale: float | None = None, row_chunk: int = 1024,
                     bias: torch.Tensor | None = None):
    """q [B, Hq, Sq, D]; k, v [B, Hkv, Skv, D] -> (o fp32 [B, Hq, Sq, D], lse fp32 [B, Hq, Sq])."""
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    bv = _bias_view(bias, B, Hq, Sq, Skv)
    out = torch.zeros((B, Hq, Sq, D), dtype=torch.float32)
    lse = torch.full((B, Hq, Sq), float("-inf"), dtype=torch.float32)
    key_pos = torch.arange(Skv).view(1, 1, Skv)
    for b in range(B):
        for kvh in range(Hkv):
            hs = slice(kvh * G, (kvh + 1) * G)
            kk = k[b, kvh].float()
            vv = v[b, kvh].float()
            qg = q[b, hs].float()  # [G, Sq, D]
            for i0 in range(0, Sq, row_chunk):
                i1 = min(Sq, i0 + row_chunk)
                s = torch.matmul(qg[:, i0:i1], kk.t()) * scale  # [G, rows, Skv]
                if bv is not None:
                    s = s + bv[b, hs, i0:i1]
                q_pos = torch.arange(i0, i1).view(1, -1, 1) + q_offset
                s = s.masked_fill(key_pos > q_pos, float("-inf"))
                p, row_lse = _softmax_rows(s)
                out[b, hs, i0:i1] = torch.matmul(p, vv)
                lse[b, hs, i0:i1] = row_lse
    return out, lse


def causal_attention_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, do: torch.Tensor,
                              q_offset: int = 0, scale: float | None = None,
                              row_chunk: int = 1024, bias: torch.Tensor | None = None):
    """Gradients of causal_attention's output O with respect to q, k, v, given dO.

    Follows the reference's backward (kernels/triton/attention.py:180-320,
    380-454): P = exp(s - lse) with s = q k^T * scale (causal, plus the
    additive bias), delta = rowsum(dO * O), dP = dO v^T, dS = P * (dP - delta),
    dq = dS k * scale, dk = dS^T q * scale, dv = P^T dO; under GQA, dk/dv sum
    over the G query heads that read kv head h // G. The bias gets no
    gradient. Shapes as causal_attention; all fp32.
    """
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    bv = _bias_view(bias, B, Hq, Sq, Skv)
    o, lse = causal_attention(q, k, v, q_offset=q_offset, scale=scale, row_chunk=row_chunk,
                              bias=bias)
    dq = torch.zeros((B, Hq, Sq, D), dtype=torch.float32)
    dk = torch.zeros((B, Hkv, Skv, D), dtype=torch.float32)
    dv = torch.zeros((B, Hkv, Skv, D), dtype=torch.float32)
    key_pos = torch.arange(Skv).view(1, 1, Skv)
    for b in range(B):
        for kvh in range(Hkv):
            kk = k[b, kvh].float()
            vv = v[b, kvh].float()
            hs = slice(kvh * G, (kvh + 1) * G)
            qg = q[b, hs].float()
            dog = do[b, hs].float()
            delta = (dog * o[b, hs]).sum(-1)  # [G, Sq]
            for i0 in range(0, Sq, row_chunk):
                i1 = min(Sq, i0 + row_chunk)
                s = torch.matmul(qg[:, i0:i1], kk.t()) * scale
                if bv is not None:
                    s = s + bv[b, hs, i0:i1]
                q_pos = torch.arange(i0, i1).view(1, -1, 1) + q_offset
                row_lse = lse[b, hs, i0:i1].unsqueeze(-1)
                ok = torch.isfinite(row_lse)
                p = torch.exp(s - torch.where(ok, row_lse, torch.zeros_like(row_lse)))
                p = torch.where((key_pos > q_pos) | ~ok, torch.zeros_like(p), p)
                dp = torch.matmul(dog[:, i0:i1], vv.t())
                ds = p * (dp - delta[:, i0:i1].unsqueeze(-1))
                dq[b, hs, i0:i1] = torch.matmul(ds, kk) * scale
                dk[b, kvh] += torch.einsum("gij,gid->jd", ds, qg[:, i0:i1]) * scale
                dv[b, kvh] += torch.einsum("gij,gid->jd", p, dog[:, i0:i1])
    return dq, dk, dv
