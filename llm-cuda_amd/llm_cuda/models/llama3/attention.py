"""Llama-3 attention (reference: models/llama3/attention.py:1-150).

Same module, parameters and call signature as the reference. The forward pass
differs only in how the attention itself is computed, all on HIP kernels:

  * Inference projections: q, k and v come out of one GEMM against the
    concatenated weight (the parameters alias its row blocks). With at most
    32 rows (a decode step) that GEMM and o_proj are native launches that
    stream the weight once (`decode_linear`).
  * RoPE: Q and K rotated in one launch, reading the transposed projection
    views directly. The cos/sin tables are built once for a range of
    positions and sliced per call (every row depends only on its position,
    so the slices equal the per-call tables of rotary.py:29-71).
  * Paged cache, one query token (decode): new K/V are scattered into the page
    pools and the query attends to the pools in place through the block table.
    For a batch of equal lengths that fills the CUs, RoPE, the append and the
    attention are one launch (one workgroup per sequence and head group);
    otherwise RoPE + append is one launch and split-K flash-decode another.
    The reference instead copied the whole cache into a contiguous tensor
    every step (kv_cache.py:65-83) and decoded that.
  * Prompt / multi-token chunk: causal prefill attention with native GQA (no
    repeated K/V) and the causal diagonal shifted by the cached prefix length,
    which covers both the reference's fused path (past_len == 0) and its
    `_torch_attention` path with `past_len` (attention.py:63-89,144-147).
  * An additive attention_mask (broadcastable to [B, H, q_len, kv_len], as the
    reference adds it to the scores, attention.py:85-86) goes into the same
    kernels: the prefill kernel for prompts and chunks, the paged decode
    kernel for one token against the paged cache, and the prefill kernel at
    the cached offset for one token against a tuple cache.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from llm_cuda.kernels import _ops
from llm_cuda.kernels.triton.attention import triton_fused_causal_attention
from llm_cuda.kernels.triton.decode_attention import (
    paged_decode_attention,
    triton_decode_attention,
)

from .config import Llama3Config
from .fused import FusedLinearWeights
from .kv_cache import PagedKVLayerCache
from .rotary import apply_rotary, build_inv_freq, build_rope_cache


class Llama3Attention(nn.Module):
    def __init__(self, config: Llama3Config):
        super().__init__()
        if config.tensor_parallel_size > 1:
            raise NotImplementedError("tensor parallelism is not part of this build")
        self.config = config
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.num_kv_groups = self.num_heads // self.num_kv_heads

        q_size = self.num_heads * self.head_dim
        kv_size = self.num_kv_heads * self.head_dim
        self.q_proj = nn.Linear(config.hidden_size, q_size, bias=False)
        self.k_proj = nn.Linear(config.hidden_size, kv_size, bias=False)
        self.v_proj = nn.Linear(config.hidden_size, kv_size, bias=False)
        self.o_proj = nn.Linear(q_size, config.hidden_size, bias=False)

        # Non-persistent buffer, like the reference: it follows the module's
        # dtype, so a bf16 model builds its RoPE tables from a bf16 inv_freq.
        inv_freq = build_inv_freq(
            head_dim=config.head_dim, base=config.rope_theta, device=torch.device("cpu"))
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        self._qkv = FusedLinearWeights(self.q_proj, self.k_proj, self.v_proj)
        self._rope_cache: tuple | None = None

    def _rope_tables(self, past_len: int, seq_len: int, device: torch.device,
                     dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        """cos, sin [seq_len, D] for positions past_len .. +seq_len-1, sliced from a
        table over positions 0 .. cap-1 (rebuilt when inv_freq, the device or the
        dtype change, and doubled when a position falls outside it)."""
        need = past_len + seq_len
        inv = self.inv_freq
        key = (inv.data_ptr(), inv._version, inv.dtype, device, dtype)
        cache = self._rope_cache
        if cache is None or cache[0] != key or cache[1] < need:
            cap = max(need, 256, 2 * cache[1] if cache is not None and cache[0] == key else 0)
            cap = 1 << (cap - 1).bit_length()
            cos, sin = build_rope_cache(
                seq_len=cap, head_dim=self.head_dim, base=self.config.rope_theta,
                device=device, dtype=dtype, position_offset=0, inv_freq=inv)
            cache = self._rope_cache = (key, cap, cos, sin)
        return cache[2][past_len:need], cache[3][past_len:need]

    def _check_mask(self, mask: torch.Tensor, bsz: int, q_len: int, kv_len: int) -> None:
        """The reference adds the mask to scores [B, H, q_len, kv_len]
        (attention.py:85-86): refuse what that add would refuse."""
        try:
            shape = torch.broadcast_shapes(tuple(mask.shape), (bsz, self.num_heads, q_len, kv_len))
        except RuntimeError as exc:
            raise ValueError(f"attention_mask of shape {tuple(mask.shape)} does not broadcast to "
                             f"{(bsz, self.num_heads, q_len, kv_len)}") from exc
        if shape != (bsz, self.num_heads, q_len, kv_len):
            raise ValueError(f"attention_mask of shape {tuple(mask.shape)} does not broadcast to "
                             f"{(bsz, self.num_heads, q_len, kv_len)}")

    def _shape(self, x: torch.Tensor, heads: int) -> torch.Tensor:
        bsz, seq_len, _ = x.shape
        return x.view(bsz, seq_len, heads, self.head_dim).transpose(1, 2)

    def forward(
        self,
        x: torch.Tensor,
        attention_mask: torch.Tensor | None = None,
        past_key_value: tuple[torch.Tensor, torch.Tensor] | PagedKVLayerCache | None = None,
        use_cache: bool = False,
        partial_out: bool = False,
    ) -> tuple[torch.Tensor, tuple[torch.Tensor, torch.Tensor] | PagedKVLayerCache | None]:
        """The reference's forward (attention.py:91-150). partial_out (an
        extension, default off): at a decode step whose o_proj runs on the
        native projection kernel, return its output as an `_ops.PartialSum`
        (split-K partials) for `add_rms_norm` to add up."""
        bsz, seq_len, _ = x.shape

        if FusedLinearWeights.usable(self.q_proj, self.k_proj, self.v_proj):
            nq, nk, _ = self._qkv.sizes()
            w = self._qkv.weight()
            qkv = _ops.decode_linear(x, w) if _ops.decode_linear_applies(x, w) else F.linear(x, w)
            q = self._shape(qkv[..., :nq], self.num_heads)
            k = self._shape(qkv[..., nq:nq + nk], self.num_kv_heads)
            v = self._shape(qkv[..., nq + nk:], self.num_kv_heads)
        else:
            q = self._shape(self.q_proj(x), self.num_heads)
            k = self._shape(self.k_proj(x), self.num_kv_heads)
            v = self._shape(self.v_proj(x), self.num_kv_heads)

        paged = isinstance(past_key_value, PagedKVLayerCache)
        if paged:
            past_len = past_key_value.length
        elif past_key_value is not None:
            past_len = past_key_value[0].shape[-2]
        else:
            past_len = 0

        if paged and use_cache and seq_len == 1:
            # Decode step, positions taken from the cache's device-side lengths:
            # RoPE, the cache append and the attention in one launch where the
            # one-workgroup-per-sequence kernel suits the batch, else RoPE and
            # the append in one launch and split-K decode in another.
            cache = past_key_value
            if attention_mask is not None:
                self._check_mask(attention_mask, bsz, 1, past_len + 1)
            rows = cache.max_pages * cache.page_size
            self._rope_tables(0, rows, x.device, x.dtype)
            cos_t, sin_t = self._rope_cache[2], self._rope_cache[3]
            if cache.can_fuse_decode_step(self.num_heads, q.dtype):
                out = cache.decode_step(q, k, v, cos_t, sin_t, attention_mask=attention_mask)
            else:
                q = cache.append_rotated(q, k, v, cos_t, sin_t)
                out = paged_decode_attention(
                    q, cache.key_pages, cache.value_pages, cache.block_table, cache.seq_lens,
                    attention_mask=attention_mask, uniform_length=cache.uniform_length)
            out = out.transpose(1, 2).reshape(bsz, seq_len, self.num_heads * self.head_dim)
            wo = self.o_proj.weight
            if partial_out and _ops.decode_linear_partials_applies(out, wo):
                return _ops.decode_linear_partials(out, wo), cache
            if _ops.decode_linear_applies(out, wo):
                return _ops.decode_linear(out, wo), cache
            return self.o_proj(out), cache

        cos, sin = self._rope_tables(past_len, seq_len, x.device, x.dtype)
        q, k = apply_rotary(q, k, cos, sin)

        mask = attention_mask
        if paged:
            cache = past_key_value
            if use_cache:
                cache.append(k, v)
            present = cache if use_cache else None
            if mask is not None:
                self._check_mask(mask, bsz, seq_len, cache.length if use_cache else past_len)
            if seq_len == 1:
                # The reference attends to get_kv(): the cache after the
                # append (or without the new token when use_cache is False).
                if cache.length == 0:
                    raise ValueError("decode step against an empty cache")
                out = paged_decode_attention(
                    q, cache.key_pages, cache.value_pages, cache.block_table, cache.seq_lens,
                    attention_mask=mask, uniform_length=cache.uniform_length)
            elif use_cache and past_len == 0:
                out = triton_fused_causal_attention(q, k, v, attention_mask=mask)
            else:
                k_all, v_all = cache.get_kv()
                out = triton_fused_causal_attention(q, k_all, v_all, attention_mask=mask,
                                                    q_offset=past_len)
        else:
            if past_key_value is not None:
                past_k, past_v = past_key_value
                k = torch.cat([past_k, k], dim=-2)
                v = torch.cat([past_v, v], dim=-2)
            present = (k, v) if use_cache else None
            if mask is not None:
                self._check_mask(mask, bsz, seq_len, k.shape[-2])
            if seq_len == 1 and past_len > 0 and mask is None:
                out = triton_decode_attention(q, k, v)
            else:
                out = triton_fused_causal_attention(q, k, v, attention_mask=mask,
                                                    q_offset=past_len)

        out = out.transpose(1, 2).reshape(bsz, seq_len, self.num_heads * self.head_dim)
        return self.o_proj(out), present

