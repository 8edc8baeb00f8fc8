"""Llama 3 model package."""

from .config import Llama3Config
from .kv_cache import PagedKVCache, PagedKVLayerCache
from .model import Llama3ForCausalLM

__all__ = ["Llama3Config", "Llama3ForCausalLM", "PagedKVCache", "PagedKVLayerCache"]
