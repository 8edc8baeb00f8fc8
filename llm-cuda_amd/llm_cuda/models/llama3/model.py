"""Llama-3 decoder stack and causal LM (reference: models/llama3/model.py:1-218).

Module structure, parameter names, initialisation (normal(0, initializer_range)
for every Linear and Embedding, reference model.py:120-139) and the greedy
`generate` loop follow the reference. `generate(use_paged_kv=True)` accepts a
batch of any size (the reference's paged cache was batch-1 only). The loss
path uses torch's cross entropy (the fused Triton cross entropy of the
reference is outside the attention path); activation checkpointing is a
training feature and is not provided.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from llm_cuda.kernels._ops import add_rms_norm, lm_head_argmax

from .attention import Llama3Attention
from .config import Llama3Config
from .kv_cache import PagedKVCache, PagedKVLayerCache
from .mlp import Llama3MLP
from .norm import RMSNorm


class Llama3DecoderLayer(nn.Module):
    def __init__(self, config: Llama3Config):
        super().__init__()
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.self_attn = Llama3Attention(config)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.mlp = Llama3MLP(config)

    def forward(
        self,
        x: torch.Tensor,
        attention_mask: torch.Tensor | None = None,
        past_key_value: tuple[torch.Tensor, torch.Tensor] | PagedKVLayerCache | None = None,
        use_cache: bool = False,
    ) -> tuple[torch.Tensor, tuple[torch.Tensor, torch.Tensor] | PagedKVLayerCache | None]:
        x, mlp_out, present = self.forward_split(
            x, None, attention_mask=attention_mask, past_key_value=past_key_value,
            use_cache=use_cache)
        return x + mlp_out, present

    def forward_split(
        self,
        x: torch.Tensor,
        pending: torch.Tensor | None,
        attention_mask: torch.Tensor | None = None,
        past_key_value: tuple[torch.Tensor, torch.Tensor] | PagedKVLayerCache | None = None,
        use_cache: bool = False,
        partial_out: bool = False,
    ):
        """The layer with its last residual add left to the caller.

        The layer's input is x + pending (pending None: x). Returns (x_mid,
        mlp_out, present) with the layer's output = x_mid + mlp_out, so that a
        stack can fuse that add with the next layer's input norm. Each add is
        rounded to x's dtype and normalised exactly as the separate add and
        norm of the reference layer (model.py:29-42). With partial_out, a
        decode step's o_proj and down_proj outputs may be `_ops.PartialSum`s
        (pending may be one too): their split-K sums are formed by the add +
        norm that consumes them, with the same value.
        """
        norm_in = self.input_layernorm
        if pending is None:
            h = norm_in(x)
        else:
            h, x = add_rms_norm(x, pending, norm_in.weight, norm_in.eps)
        attn_out, present = self.self_attn(
            h, attention_mask=attention_mask, past_key_value=past_key_value, use_cache=use_cache,
            partial_out=partial_out)
        norm_post = self.post_attention_layernorm
        h, x = add_rms_norm(x, attn_out, norm_post.weight, norm_post.eps)
        return x, self.mlp(h, partial_out=partial_out), present


class Llama3Model(nn.Module):
    def __init__(self, config: Llama3Config):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(
            [Llama3DecoderLayer(config) for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(
        self,
        input_ids: torch.Tensor,
        attention_mask: torch.Tensor | None = None,
        past_key_values: list[tuple[torch.Tensor, torch.Tensor]] | PagedKVCache | None = None,
        use_cache: bool = False,
    ) -> dict:
        x = self.embed_tokens(input_ids)
        paged = isinstance(past_key_values, PagedKVCache)
        presents: list[tuple[torch.Tensor, torch.Tensor]] = []
        # Each layer's closing residual add is fused with the next norm (the
        # next layer's input norm, or the final norm): `pending` carries the
        # MLP output still to be added to x (at a decode step, its split-K
        # partials: the add + norm forms their sum).
        pending = None
        for idx, layer in enumerate(self.layers):
            if paged:
                layer_past = past_key_values.get_layer(idx)
            else:
                layer_past = None if past_key_values is None else past_key_values[idx]
            x, pending, present = layer.forward_split(
                x, pending, attention_mask=attention_mask, past_key_value=layer_past,
                use_cache=use_cache, partial_out=True)
            if use_cache and not paged and present is not None:
                presents.append(present)
        if pending is None:
            x = self.norm(x)
        else:
            x, _ = add_rms_norm(x, pending, self.norm.weight, self.norm.eps)
        if paged:
            next_cache = past_key_values if use_cache else None
        else:
            next_cache = presents if use_cache else None
        return {"hidden_states": x, "past_key_values": next_cache}


class Llama3ForCausalLM(nn.Module):
    def __init__(self, config: Llama3Config):
        super().__init__()
        self.config = config
        self.model = Llama3Model(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        self.apply(self._init_weights)

    def _init_weights(self, module: nn.Module) -> None:
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)

    def forward(
        self,
        input_ids: torch.Tensor,
        attention_mask: torch.Tensor | None = None,
        labels: torch.Tensor | None = None,
        past_key_values: list[tuple[torch.Tensor, torch.Tensor]] | PagedKVCache | None = None,
        use_cache: bool = False,
    ) -> dict:
        model_out = self.model(
            input_ids,
            attention_mask=attention_mask,
            past_key_values=past_key_values,
            use_cache=use_cache,
        )
        logits = self.lm_head(model_out["hidden_states"])
        loss = None
        if labels is not None:
            shift_logits = logits[:, :-1, :].reshape(-1, self.config.vocab_size)
            shift_labels = labels[:, 1:].reshape(-1)
            loss = F.cross_entropy(shift_logits.float(), shift_labels, ignore_index=-100)
        return {"logits": logits, "loss": loss, "past_key_values": model_out["past_key_values"]}

    @torch.no_grad()
    def generate(
        self,
        input_ids: torch.Tensor,
        max_new_tokens: int = 16,
        use_paged_kv: bool = False,
        page_size: int = 64,
        use_graph: bool = False,
    ) -> torch.Tensor:
        """Greedy decoding; returns prompt + max_new_tokens ids.

        use_graph (an extension, default off; needs use_paged_kv): the prompt
        and the first decode step run eagerly, the next decode step is
        captured in a HIP graph and every later token replays it. The captured
        kernels take the positions from the cache's device-side lengths, which
        each replay advances, so the replays give the eager loop's ids; the
        launch cost of a step (a few hundred kernels at the 8B shape) is paid
        once instead of per token.
        """
        if use_graph and not use_paged_kv:
            raise ValueError("use_graph needs use_paged_kv=True (the tuple cache grows by "
                             "concatenation, which a captured graph cannot replay)")
        self.eval()
        generated = input_ids
        if use_paged_kv:
            past_key_values = PagedKVCache.create(
                num_layers=self.config.num_hidden_layers,
                num_kv_heads=self.config.num_key_value_heads,
                head_dim=self.config.head_dim,
                max_seq_len=input_ids.shape[1] + max_new_tokens,
                page_size=page_size,
                device=input_ids.device,
                dtype=self.model.embed_tokens.weight.dtype,
                batch_size=input_ids.shape[0],
            )
        else:
            past_key_values = None
        cur_input = input_ids
        eager_steps = min(max_new_tokens, 2) if use_graph else max_new_tokens
        for _ in range(eager_steps):
            next_token, past_key_values = self.greedy_next_token(cur_input, past_key_values)
            generated = torch.cat([generated, next_token], dim=1)
            cur_input = next_token
        if eager_steps == max_new_tokens:
            return generated
        # The eager decode step above allocated what the step needs (counters,
        # workspaces, tables), so the capture records kernels only. Capturing
        # runs no kernel: the host-side lengths advance once here while the
        # device-side ones advance with every replay.
        static_in = cur_input.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_out, _ = self.greedy_next_token(static_in, past_key_values)
        for _ in range(max_new_tokens - eager_steps):
            graph.replay()
            next_token = static_out.clone()
            generated = torch.cat([generated, next_token], dim=1)
            static_in.copy_(next_token)
        final = input_ids.shape[1] + max_new_tokens - 1
        for layer in past_key_values.layer_caches:
            layer.lengths = [final] * layer.batch_size
        return generated

    @torch.no_grad()
    def greedy_next_token(self, input_ids: torch.Tensor, past_key_values=None,
                          return_logit: bool = False):
        """argmax of the last position's logits, [B, 1] int64, and the cache.

        The reference computes lm_head over every position and then takes
        torch.argmax(logits[:, -1, :]) (model.py:156,214); here the lm_head
        projection and the argmax run as one kernel on the last position only,
        with the same result (logits rounded to the model dtype, first index on
        ties) and without writing the [B, V] logits. With return_logit, the
        winning logit (fp32 [B]) is returned as a third value.
        """
        out = self.model(input_ids, past_key_values=past_key_values, use_cache=True)
        hidden = out["hidden_states"][:, -1, :]
        ids, best = lm_head_argmax(hidden, self.lm_head.weight, return_max=True)
        if return_logit:
            return ids.unsqueeze(-1), out["past_key_values"], best
        return ids.unsqueeze(-1), out["past_key_values"]
