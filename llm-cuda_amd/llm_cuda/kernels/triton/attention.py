"""Causal prefill attention entry (reference: kernels/triton/attention.py:480-535).

`triton_fused_causal_attention(q, k, v, attention_mask)` computes
softmax(q k^T / sqrt(D) + causal + attention_mask) v on the lc_prefill_attn_fwd
HIP kernel. Differences from the
reference, all widening the accepted inputs:
  * GQA is native: k and v may carry fewer heads than q (n_heads a multiple
    of n_kv_heads); the reference required q.shape == k.shape and its callers
    materialised the repeated K/V (models/llama3/attention.py:141-142).
  * `return_lse=True` also returns the fp32 natural-log logsumexp [B, H, S]
    (the reference kept it internal, attention.py:330-333).
  * `q_offset` shifts the causal diagonal for queries that continue a cached
    prefix (key j is visible to query i iff j <= i + q_offset), the masking of
    models/llama3/attention.py:63-89.
  * `attention_mask`, the reference's additive mask (broadcastable to
    [B, H, Sq, Skv], fp32 or q's dtype), is added to the scaled scores inside
    the kernel, as the reference's torch path does (attention.py:457-477). A
    row whose visible keys are all at -inf gives zeros (the reference: NaN).

Autograd: when any of q, k, v requires grad, the call goes through
`_FusedCausalAttentionFunction` (reference: attention.py:323-454), whose
backward runs lc_prefill_attn_bwd on the saved q, k, v, output, logsumexp and
mask. The returned lse and the mask get no gradient (a mask that requires
grad is refused).
"""
from __future__ import annotations

import torch

from llm_cuda.kernels import _ops


def _select_attention_block_sizes(seq_len: int, head_dim: int) -> tuple[int, int]:
    """(keys per tile, padded head_dim) of the reference's Triton tiling policy
    (kernels/triton/attention.py:16-29): 32 / 64 / 128 keys from sequence
    lengths 256 and 1024 up, head_dim rounded up to a power of two in [16, 128].

    Kept for callers and tests that query it. The HIP kernels do not consult
    it: the MFMA kernel's tiles are fixed at 64 keys x head_dim padded to 64
    or 128, the generic kernel's at 16 keys.
    """
    if seq_len >= 1024:
        block_n = 128
    elif seq_len >= 256:
        block_n = 64
    else:
        block_n = 32
    block_d = 1 << max(0, int(head_dim) - 1).bit_length()
    return block_n, min(max(block_d, 16), 128)


def _select_attention_num_warps(head_dim: int, block_n: int) -> int:
    """Warp count of the reference's Triton policy (attention.py:32-38), by the
    tile's head_dim x keys work: 8 from 8192, 4 from 4096, else 2. Kept for
    callers that query it; no HIP launch depends on it."""
    work = int(head_dim) * int(block_n)
    return 8 if work >= 8192 else (4 if work >= 4096 else 2)


def _should_use_cuda_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          attention_mask: torch.Tensor | None = None) -> bool:
    """Whether a call would be routed to torch SDPA (reference attention.py:41-58).

    Always False here: this build has no SDPA branch, every eligible call runs
    the gfx950 MFMA kernel (on host tensors the reference also answers False).
    """
    return False


def _cuda_sdpa_causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Causal attention of q, k, v [B, H, S, D] with scale 1/sqrt(D) and no mask
    (reference: attention.py:61-69, which calls torch SDPA with is_causal=True).

    Kept under the reference's name for callers that import or patch it; here
    it runs the same gfx950 MFMA kernel as triton_fused_causal_attention (GQA
    k/v with fewer heads are taken as well), so no second attention path
    exists. Forward only, like the rest of the dispatcher's non-autograd path.
    """
    if not _gqa_compatible(q, k, v):
        raise ValueError("q, k, v must be [batch, heads, seq, head_dim] with n_heads a "
                         "multiple of n_kv_heads")
    return _ops.prefill_attention(q, k, v)


def _gqa_compatible(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or k.shape != v.shape:
        return False
    if q.shape[0] != k.shape[0] or q.shape[3] != k.shape[3]:
        return False
    return k.shape[1] > 0 and q.shape[1] % k.shape[1] == 0


def can_use_triton_fused_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    attention_mask: torch.Tensor | None = None,
) -> bool:
    """Whether the HIP kernel takes the call (reference predicate: attention.py:
    480-498). Additive float masks on the same device are taken as well."""
    if attention_mask is not None and not (attention_mask.is_floating_point()
                                           and attention_mask.device == q.device):
        return False
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return False
    if not _gqa_compatible(q, k, v):
        return False
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    if not (q.dtype == k.dtype == v.dtype):
        return False
    if q.shape[-1] > 256:
        return False
    return True


class _FusedCausalAttentionFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, q_offset: int, mask):
        out, lse = _ops.prefill_attention(q, k, v, q_offset=q_offset, return_lse=True,
                                          attention_mask=mask)
        ctx.save_for_backward(q, k, v, out, lse, mask)
        ctx.q_offset = q_offset
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        q, k, v, out, lse, mask = ctx.saved_tensors
        if dout is None:
            dout = torch.zeros_like(out)
        dq, dk, dv = _ops.prefill_attention_backward(q, k, v, out, lse, dout,
                                                     q_offset=ctx.q_offset, attention_mask=mask)
        return dq, dk, dv, None, None


def triton_fused_causal_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    attention_mask: torch.Tensor | None = None,
    *,
    return_lse: bool = False,
    q_offset: int = 0,
):
    """Causal attention for q [B, Hq, S, D], k/v [B, Hkv, Skv, D] with an optional
    additive attention_mask (reference: kernels/triton/attention.py:501-535)."""
    if not _gqa_compatible(q, k, v):
        raise ValueError(
            "q, k, v must be [batch, heads, seq, head_dim] with matching batch/head_dim and "
            "n_heads a multiple of n_kv_heads")
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        if attention_mask is not None and attention_mask.requires_grad:
            raise NotImplementedError(
                "attention_mask requires grad; the HIP backward gives the mask no gradient")
        out, lse = _FusedCausalAttentionFunction.apply(q, k, v, int(q_offset), attention_mask)
        return (out, lse) if return_lse else out
    return _ops.prefill_attention(q, k, v, q_offset=q_offset, return_lse=return_lse,
                                  attention_mask=attention_mask)
