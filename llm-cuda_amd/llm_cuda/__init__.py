"""llm_cuda: the Llama-3 inference attention path on hand-written gfx950 (MI355X) kernels."""

from .models.llama3.config import Llama3Config
from .models.llama3.kv_cache import PagedKVCache, PagedKVLayerCache
from .models.llama3.model import Llama3ForCausalLM

__all__ = ["Llama3Config", "Llama3ForCausalLM", "PagedKVCache", "PagedKVLayerCache"]
