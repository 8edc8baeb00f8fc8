"""Greedy next-token oracle: lm_head projection + argmax. TEST INFRASTRUCTURE ONLY.

Follows the reference's decode step: logits = self.lm_head(hidden_states)
(models/llama3/model.py:156), an nn.Linear whose output is in the model dtype,
then next_token = torch.argmax(logits[:, -1, :], dim=-1) (model.py:214).
"""
from __future__ import annotations

import torch


def lm_head_logits(hidden: torch.Tensor, weight: torch.Tensor,
                   acc_dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """hidden [B, K] . weight[V, K]^T accumulated in acc_dtype, rounded once to
    hidden's dtype (the dtype of the reference's lm_head output), on the host."""
    h = hidden.detach().to("cpu", acc_dtype)
    w = weight.detach().to("cpu", acc_dtype)
    return (h @ w.t()).to(hidden.dtype)


def argmax_first(logits: torch.Tensor) -> torch.Tensor:
    """torch.argmax over the last dim with its documented tie rule (first
    maximal index) and NaN ranking above every number (first NaN wins)."""
    x = logits.detach().to("cpu", torch.float64)
    nan = torch.isnan(x)
    has_nan = nan.any(dim=-1)
    first_nan = torch.argmax(nan.to(torch.int8), dim=-1)
    filled = torch.where(nan, torch.full_like(x, -float("inf")), x)
    mx = filled.max(dim=-1, keepdim=True).values
    first_max = torch.argmax((filled == mx).to(torch.int8), dim=-1)
    return torch.where(has_nan, first_nan, first_max)


def lm_head_argmax(hidden: torch.Tensor, weight: torch.Tensor,
                   acc_dtype: torch.dtype = torch.float64):
    """(ids [B] int64, winning logit [B] fp32, rounded logits [B, V])."""
    logits = lm_head_logits(hidden, weight, acc_dtype)
    ids = argmax_first(logits)
    best = logits.float().gather(-1, ids.view(-1, 1)).view(-1)
    return ids, best, logits
