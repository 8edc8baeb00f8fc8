"""Paged KV cache with a real block table (reference: models/llama3/kv_cache.py:1-125).

Layout (unchanged from the reference): per layer, `key_pages` and
`value_pages` are pools [num_pages, n_kv_heads, page_size, head_dim] in the
model dtype; token t of a sequence lives in page t // page_size, slot
t % page_size of that sequence's pages. What changes:
  * `block_table` (int32 [batch, max_pages]) maps each sequence's logical page
    to a physical page of the pool. The default table gives sequence b the
    pages b*max_pages .. (b+1)*max_pages - 1, so for batch 1 logical page i IS
    physical page i, the reference's identity mapping (kv_cache.py:55-57).
  * batch > 1 and per-sequence lengths (`seq_lens`, int32 [batch] on the
    device, mirrored on the host in `lengths`).
  * `append` is one HIP scatter launch (lc_paged_kv_append) instead of a Python
    loop of 2*seq slice copies; `get_kv` is one HIP gather (lc_paged_kv_gather)
    instead of a torch.cat of pages. The decode path does not call get_kv at
    all: it reads the pools in place (paged_decode_attention).
"""
from __future__ import annotations

import math

import torch

from llm_cuda.kernels import _ops


class PagedKVLayerCache:
    def __init__(
        self,
        num_kv_heads: int,
        head_dim: int,
        max_seq_len: int,
        page_size: int,
        device: torch.device,
        dtype: torch.dtype,
        batch_size: int = 1,
        block_table: torch.Tensor | None = None,
        num_pages: int | None = None,
        seq_lens: torch.Tensor | None = None,
    ):
        if page_size <= 0:
            raise ValueError("page_size must be > 0")
        if max_seq_len <= 0:
            raise ValueError("max_seq_len must be > 0")
        if batch_size <= 0:
            raise ValueError("batch_size must be > 0")

        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.page_size = page_size
        self.batch_size = batch_size
        self.max_pages = math.ceil(max_seq_len / page_size)
        device = torch.device(device)

        if block_table is None:
            pool = batch_size * self.max_pages if num_pages is None else num_pages
            if pool < batch_size * self.max_pages:
                raise ValueError("num_pages too small for the default block table")
            block_table = torch.arange(
                batch_size * self.max_pages, dtype=torch.int32, device=device
            ).view(batch_size, self.max_pages)
        else:
            if block_table.dtype != torch.int32 or block_table.shape != (batch_size, self.max_pages):
                raise ValueError(
                    f"block_table must be int32 [{batch_size}, {self.max_pages}]")
            block_table = block_table.to(device).contiguous()
            pool = int(block_table.max().item()) + 1 if num_pages is None else num_pages
        self.num_pages = pool
        self.block_table = block_table

        self.key_pages = torch.empty(
            pool, num_kv_heads, page_size, head_dim, device=device, dtype=dtype)
        self.value_pages = torch.empty_like(self.key_pages)
        if seq_lens is None:
            seq_lens = torch.zeros(batch_size, dtype=torch.int32, device=device)
        elif (seq_lens.dtype != torch.int32 or seq_lens.shape != (batch_size,)
              or seq_lens.device != device):
            raise ValueError(f"seq_lens must be int32 [{batch_size}] on {device}")
        else:
            seq_lens.zero_()
        self.seq_lens = seq_lens
        self.lengths = [0] * batch_size
        # Zeroed scratch of the fused decode step (it leaves the counters at zero).
        self.step_counters = torch.zeros(batch_size, dtype=torch.int32, device=device)

    @property
    def length(self) -> int:
        """Cached tokens per sequence (all sequences advance together in `append`)."""
        first = self.lengths[0]
        if any(n != first for n in self.lengths):
            raise ValueError("sequences have different lengths; use `lengths`")
        return first

    @property
    def uniform_length(self) -> int | None:
        """The common number of cached tokens when every sequence holds the
        same number (host mirror), else None."""
        first = self.lengths[0]
        return first if all(n == first for n in self.lengths) else None

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        if k.shape != v.shape:
            raise ValueError("k and v shapes must match")
        if k.dim() != 4:
            raise ValueError("Expected k/v shape [batch, kv_heads, seq, head_dim]")
        if k.shape[0] != self.batch_size:
            raise ValueError(
                f"batch {k.shape[0]} does not match the cache batch size {self.batch_size}")
        if k.shape[1] != self.num_kv_heads or k.shape[3] != self.head_dim:
            raise ValueError("k/v shapes do not match cache layout")
        seq = k.shape[2]
        if max(self.lengths) + seq > self.max_seq_len:
            raise ValueError("Appending would exceed max_seq_len")
        if seq == 0:
            return
        _ops.kv_append(k, v, self.key_pages, self.value_pages, self.block_table, self.seq_lens)
        self.seq_lens.add_(seq)
        self.lengths = [n + seq for n in self.lengths]

    def append_rotated(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        """Decode-time fusion of RoPE and `append`: rotates q and k at the
        positions seq_lens[b] + s, appends the rotated k and v, and returns the
        rotated q. cos/sin are full tables indexed by position that cover
        max_pages * page_size positions."""
        if k.shape != v.shape or k.dim() != 4 or q.dim() != 4:
            raise ValueError("Expected q, k, v of shape [batch, heads, seq, head_dim]")
        if k.shape[0] != self.batch_size or q.shape[0] != self.batch_size:
            raise ValueError(
                f"batch {k.shape[0]} does not match the cache batch size {self.batch_size}")
        if k.shape[1] != self.num_kv_heads or k.shape[3] != self.head_dim:
            raise ValueError("k/v shapes do not match cache layout")
        seq = k.shape[2]
        if max(self.lengths) + seq > self.max_seq_len:
            raise ValueError("Appending would exceed max_seq_len")
        q_rot = _ops.rope_kv_append(q, k, v, cos, sin, self.key_pages, self.value_pages,
                                    self.block_table, self.seq_lens)
        self.lengths = [n + seq for n in self.lengths]
        return q_rot

    def can_fuse_decode_step(self, n_heads: int, dtype: torch.dtype) -> bool:
        """Whether `decode_step` takes this cache: equal lengths, a head layout
        whose (sequence, kv head, head group) units fill whole rounds of the
        CUs, and sizes the fused kernel supports (its single split must be
        the split the decode heuristic would choose)."""
        capacity = self.max_pages * self.page_size
        length = self.uniform_length
        if not (length is not None and self.key_pages.is_cuda
                and _ops.decode_step_supported(dtype, self.head_dim, self.page_size, capacity)):
            return False
        group = n_heads // self.num_kv_heads
        split = _ops.choose_split_tokens(
            self.batch_size, self.num_kv_heads, group, capacity, self.page_size, self.head_dim,
            length + 1, _ops._cu_count(self.key_pages.device))
        return split >= capacity

    def decode_step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor, attention_mask: torch.Tensor | None = None,
                    return_lse: bool = False):
        """One decode step of attention in one launch: RoPE of q and k at the
        positions seq_lens[b], the append of the rotated k and v, and attention
        of the rotated q over the cache including the new token. Advances the
        lengths by one and returns out [B, Hq, 1, D] (and the fp32 lse [B, Hq]
        if return_lse). cos/sin are full tables indexed by position covering
        max_pages * page_size positions."""
        if k.shape != v.shape or k.dim() != 4 or q.dim() != 4 or k.shape[2] != 1:
            raise ValueError("Expected q [batch, heads, 1, head_dim] and k, v [batch, kv_heads, "
                             "1, head_dim]")
        if k.shape[0] != self.batch_size or q.shape[0] != self.batch_size:
            raise ValueError(
                f"batch {k.shape[0]} does not match the cache batch size {self.batch_size}")
        if k.shape[1] != self.num_kv_heads or k.shape[3] != self.head_dim:
            raise ValueError("k/v shapes do not match cache layout")
        if max(self.lengths) + 1 > self.max_seq_len:
            raise ValueError("Appending would exceed max_seq_len")
        res = _ops.paged_decode_step(q, k, v, cos, sin, self.key_pages, self.value_pages,
                                     self.block_table, self.seq_lens, self.step_counters,
                                     attention_mask=attention_mask, return_lse=return_lse)
        self.lengths = [n + 1 for n in self.lengths]
        return res

    def get_kv(self) -> tuple[torch.Tensor, torch.Tensor]:
        length = self.length
        if length == 0:
            empty = self.key_pages.new_empty(
                (self.batch_size, self.num_kv_heads, 0, self.head_dim))
            return empty, empty
        return _ops.kv_gather(self.key_pages, self.value_pages, self.block_table, length)

    def clear(self) -> None:
        self.lengths = [0] * self.batch_size
        self.seq_lens.zero_()


class PagedKVCache:
    def __init__(self, layer_caches: list[PagedKVLayerCache],
                 seq_lens_all: torch.Tensor | None = None):
        if not layer_caches:
            raise ValueError("layer_caches must not be empty")
        self.layer_caches = layer_caches
        # [num_layers, batch] int32 whose rows are the layers' seq_lens when the
        # cache was made by create(): one fill resets every layer's lengths.
        self.seq_lens_all = seq_lens_all

    @classmethod
    def create(
        cls,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        max_seq_len: int,
        page_size: int,
        device: torch.device,
        dtype: torch.dtype,
        batch_size: int = 1,
        block_table: torch.Tensor | None = None,
        num_pages: int | None = None,
    ) -> "PagedKVCache":
        device = torch.device(device)
        lens = torch.zeros(num_layers, batch_size, dtype=torch.int32, device=device)
        return cls(
            [
                PagedKVLayerCache(
                    num_kv_heads=num_kv_heads,
                    head_dim=head_dim,
                    max_seq_len=max_seq_len,
                    page_size=page_size,
                    device=device,
                    dtype=dtype,
                    batch_size=batch_size,
                    block_table=block_table,
                    num_pages=num_pages,
                    seq_lens=lens[i],
                )
                for i in range(num_layers)
            ],
            seq_lens_all=lens,
        )

    def get_layer(self, layer_idx: int) -> PagedKVLayerCache:
        return self.layer_caches[layer_idx]

    def clear(self) -> None:
        for layer in self.layer_caches:
            layer.clear()
