"""Functional fp32 Llama-3 forward on the host. TEST INFRASTRUCTURE ONLY.

Restates models/llama3/model.py:22-43,54-107,141-176 (pre-norm residual
decoder layers, final norm, lm_head) and models/llama3/attention.py:91-150
(q/k/v projections, RoPE at the cached-prefix offset, causal attention with
GQA, o_proj) over a plain state dict, computing every op in fp32 from the
weights as stored. `greedy` decodes by full recomputation each step, the
invariant the reference pins its cached and paged decode against
(tests/test_llama3_shapes.py:47-88,152-198).
"""
from __future__ import annotations

import torch

from .attention import causal_attention
from .elementwise import apply_rope, build_rope_cache, rms_norm, swiglu


def _lin(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return torch.matmul(x, w.float().t())


def forward(state: dict, cfg, input_ids: torch.Tensor, rope_dtype: torch.dtype = torch.float32,
            inv_freq: torch.Tensor | None = None,
            attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Full-sequence logits [B, S, vocab] (fp32) for input_ids [B, S].

    rope_dtype / inv_freq: dtype of the RoPE tables and the inv_freq buffer of
    the model being checked (a bf16 model builds bf16 tables from a bf16
    inv_freq, reference rotary.py:61-70). attention_mask: the additive mask
    every layer adds to its scores (reference model.py:54-107 passes it to
    each layer; attention.py:85-86 adds it).
    """
    sd = {k: v.detach().cpu() for k, v in state.items()}
    ids = input_ids.cpu()
    B, S = ids.shape
    H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    x = sd["model.embed_tokens.weight"].float()[ids]
    cos, sin = build_rope_cache(S, D, cfg.rope_theta, rope_dtype, 0, inv_freq)
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        h = rms_norm(x, sd[p + "input_layernorm.weight"], cfg.rms_norm_eps)
        q = _lin(h, sd[p + "self_attn.q_proj.weight"]).view(B, S, H, D).transpose(1, 2)
        k = _lin(h, sd[p + "self_attn.k_proj.weight"]).view(B, S, Hkv, D).transpose(1, 2)
        v = _lin(h, sd[p + "self_attn.v_proj.weight"]).view(B, S, Hkv, D).transpose(1, 2)
        q = apply_rope(q, cos, sin)
        k = apply_rope(k, cos, sin)
        o, _ = causal_attention(q, k, v, bias=None if attention_mask is None else attention_mask.cpu())
        o = o.transpose(1, 2).reshape(B, S, H * D)
        x = x + _lin(o, sd[p + "self_attn.o_proj.weight"])
        h = rms_norm(x, sd[p + "post_attention_layernorm.weight"], cfg.rms_norm_eps)
        g = _lin(h, sd[p + "mlp.gate_proj.weight"])
        u = _lin(h, sd[p + "mlp.up_proj.weight"])
        x = x + _lin(swiglu(g, u), sd[p + "mlp.down_proj.weight"])
    x = rms_norm(x, sd["model.norm.weight"], cfg.rms_norm_eps)
    return _lin(x, sd["lm_head.weight"])


def greedy(state: dict, cfg, input_ids: torch.Tensor, max_new_tokens: int, **kw):
    """Greedy ids [B, S + n] and the per-step last-position logits [n, B, vocab]."""
    ids = input_ids.cpu()
    steps = []
    for _ in range(max_new_tokens):
        logits = forward(state, cfg, ids, **kw)[:, -1, :]
        steps.append(logits)
        ids = torch.cat([ids, torch.argmax(logits, dim=-1, keepdim=True)], dim=1)
    return ids, torch.stack(steps)
