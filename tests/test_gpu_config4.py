"""GPU parity at benchmark config 4: the Llama-3-8B decode step.

Shape: dim 4096, 32/8 heads, head_dim 128, FFN 14336, vocab 128256, bf16,
random init normal(0, 0.02) as reference models/llama3/model.py:122-139;
batch 32, paged KV at context 2048 (pools ~N(0,1), a seeded random
permutation of physical pages, page size 64), one new token per sequence.

Each block of the decode step is checked against the oracle's fp32
composition on the same weights, fed the HIP step's own bf16 input to that
block (so the bound is one block's rounding, not the drift of a bf16 chain).
Inside a block the oracle rounds to bf16 where the reference's bf16 modules
return bf16 (each nn.Linear output, RoPE, the attention output, SwiGLU):
  * input / post-attention add + RMSNorm: oracle.elementwise.rms_norm of the
    bf16 residual sums (reference model.py:29-42, norm.py:31-33);
  * attention: q/k/v = h W^T in fp32, RoPE at position 2048
    (oracle.elementwise.apply_rope on the model's own tables), the cached
    2048 tokens gathered through the block table (oracle.decode.gather_pages)
    plus the new token, oracle.decode.decode_attention (output and lse), then
    o_proj (reference models/llama3/attention.py:91-150). At this shape RoPE,
    the append and the attention run as one launch (lc_paged_decode_step),
    whose rotated q never leaves the kernel: its output, lse and the appended
    K/V are what is checked;
  * the K/V the step appended to the pools at position 2048;
  * MLP: down(silu(h W_g^T) * h W_u^T) (reference mlp.py:39-43);
  * the final norm and the greedy id (oracle.lm_head, reference
    model.py:156,214) from the HIP final hidden state.
The full 32-layer step also runs as a HIP graph: every replay equals the
eager step bit for bit, and the fused lm_head + argmax picks the argmax of the
step's full logits.
"""
import math

import pytest
import torch

from helpers import assert_close, assert_lse_close
from oracle.decode import decode_attention, gather_pages_torch
from oracle.elementwise import apply_rope, build_rope_cache, rms_norm, swiglu
from oracle.lm_head import lm_head_argmax as oracle_argmax

pytestmark = pytest.mark.gpu

B, CTX, P = 32, 2048, 64
BF16_ATOL, BF16_RTOL = 2e-2, 2.0 ** -7


def _config(layers):
    from llm_cuda.models.llama3.config import Llama3Config

    return Llama3Config(vocab_size=128256, hidden_size=4096, intermediate_size=14336,
                        num_hidden_layers=layers, num_attention_heads=32, num_key_value_heads=8,
                        max_position_embeddings=8192, rope_theta=500000.0)


def _build(dev, layers):
    """The config-4 model and a cache holding CTX tokens per sequence."""
    from llm_cuda.models.llama3.kv_cache import PagedKVCache
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = _config(layers)
    torch.manual_seed(0)
    with torch.device(dev):
        model = Llama3ForCausalLM(cfg)
    model = model.to(device=dev, dtype=torch.bfloat16).eval()
    max_pages = math.ceil((CTX + 1) / P)
    g = torch.Generator().manual_seed(0)
    table = torch.randperm(B * max_pages, generator=g).to(torch.int32).view(B, max_pages)
    cache = PagedKVCache.create(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                                max_pages * P, P, dev, torch.bfloat16, batch_size=B,
                                block_table=table, num_pages=B * max_pages)
    gd = torch.Generator(device=dev).manual_seed(0)
    for layer in cache.layer_caches:
        layer.key_pages.normal_(generator=gd)
        layer.value_pages.normal_(generator=gd)
    ids = torch.randint(0, cfg.vocab_size, (B, 1), generator=gd, device=dev)
    return cfg, model, cache, ids


def _reset(cache):
    cache.seq_lens_all.fill_(CTX)
    for layer in cache.layer_caches:
        layer.lengths = [CTX] * B


class _Capture:
    """Records each layer's attention and MLP inputs/outputs and the decode
    attention's rotated q (None where RoPE, the append and the attention run
    as one fused launch), output and lse during one eager step."""

    def __init__(self, model, monkeypatch):
        import llm_cuda.models.llama3.attention as attn_mod
        from llm_cuda.models.llama3.kv_cache import PagedKVLayerCache

        self.attn_in, self.attn_out, self.mlp_in, self.mlp_out = [], [], [], []
        self.dec = []
        self.fused = 0
        self.handles = []
        for layer in model.model.layers:
            self.handles.append(layer.self_attn.register_forward_hook(self._hook(
                self.attn_in, self.attn_out, tuple_out=True)))
            self.handles.append(layer.mlp.register_forward_hook(self._hook(
                self.mlp_in, self.mlp_out, tuple_out=False)))
        orig = attn_mod.paged_decode_attention

        def recording(q, kp, vp, bt, sl, **kw):
            out, lse = orig(q, kp, vp, bt, sl, return_lse=True, **kw)
            self.dec.append((q.detach().clone(), out.detach().clone(), lse.detach().clone()))
            return out

        monkeypatch.setattr(attn_mod, "paged_decode_attention", recording)
        orig_step = PagedKVLayerCache.decode_step

        def recording_step(cache, q, k, v, cos, sin, attention_mask=None):
            out, lse = orig_step(cache, q, k, v, cos, sin, attention_mask=attention_mask,
                                 return_lse=True)
            self.dec.append((None, out.detach().clone(), lse.detach().clone()))
            self.fused += 1
            return out

        monkeypatch.setattr(PagedKVLayerCache, "decode_step", recording_step)

    @staticmethod
    def _hook(ins, outs, tuple_out):
        from llm_cuda.kernels._ops import PartialSum

        def fn(mod, args, out):
            ins.append(args[0].detach().clone())
            o = out[0] if tuple_out else out
            # o_proj / down_proj outputs may be split-K partials whose sum the
            # next add + norm forms: record that value
            outs.append(o.materialize() if isinstance(o, PartialSum) else o.detach().clone())
        return fn

    def remove(self):
        for h in self.handles:
            h.remove()


def _w(mod):
    return mod.weight.detach().float().cpu()


def _bf(x):
    """Round to bf16, where the reference's bf16 modules round their outputs."""
    return x.to(torch.bfloat16).float()


def _check_layer(model, cache, cfg, cap, i, x_in, pending):
    """Checks layer i's blocks against the oracle; returns the layer's residual
    stream (x_mid, mlp_out) as the HIP step rounded it (bf16, host)."""
    layer = model.model.layers[i]
    attn = layer.self_attn
    H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps = cfg.rms_norm_eps

    # input add + norm (layer 0: the embedding alone)
    x = x_in if pending is None else (x_in + pending)  # bf16 add, as the model rounds it
    h = attn_in = cap.attn_in[i].cpu()
    assert_close(h, rms_norm(x, _w(layer.input_layernorm), eps), BF16_ATOL,
                 f"layer {i} input norm", rtol=BF16_RTOL)

    # attention block from the HIP step's normed input; intermediates are
    # rounded to bf16 where the reference's modules return bf16 (each
    # nn.Linear output, the RoPE output, the attention output)
    hf = attn_in.float()
    q = _bf((hf @ _w(attn.q_proj).t()).view(B, 1, H, D).transpose(1, 2))
    k = _bf((hf @ _w(attn.k_proj).t()).view(B, 1, Hkv, D).transpose(1, 2))
    v = _bf((hf @ _w(attn.v_proj).t()).view(B, 1, Hkv, D).transpose(1, 2))
    cos, sin = build_rope_cache(1, D, cfg.rope_theta, torch.bfloat16, position_offset=CTX,
                                inv_freq=attn.inv_freq.detach().cpu())
    q = _bf(apply_rope(q, cos, sin))
    k = _bf(apply_rope(k, cos, sin))
    lc = cache.get_layer(i)
    bt = lc.block_table.cpu()
    kp, vp = lc.key_pages.cpu(), lc.value_pages.cpu()
    # the step appended token CTX: page bt[b, CTX // P], slot CTX % P
    new_k = torch.stack([kp[int(bt[b, CTX // P]), :, CTX % P] for b in range(B)])
    new_v = torch.stack([vp[int(bt[b, CTX // P]), :, CTX % P] for b in range(B)])
    assert_close(new_k, k[:, :, 0], BF16_ATOL, f"layer {i} appended k", rtol=BF16_RTOL)
    assert_close(new_v, v[:, :, 0], BF16_ATOL, f"layer {i} appended v", rtol=BF16_RTOL)
    kk = torch.cat([gather_pages_torch(kp, bt, CTX).float(), k], dim=2)
    vv = torch.cat([gather_pages_torch(vp, bt, CTX).float(), v], dim=2)
    o, lse = decode_attention(q, kk, vv)
    dq, dout, dlse = cap.dec[i]
    if dq is not None:
        assert_close(dq, q, BF16_ATOL, f"layer {i} rotated q", rtol=BF16_RTOL)
    assert_close(dout, o, BF16_ATOL, f"layer {i} decode out")
    assert_lse_close(dlse, lse, f"layer {i} decode lse")
    a_out = _bf(o).transpose(1, 2).reshape(B, 1, H * D) @ _w(attn.o_proj).t()
    attn_out = cap.attn_out[i].cpu()
    assert_close(attn_out, a_out, BF16_ATOL, f"layer {i} attention out", rtol=BF16_RTOL)

    # post-attention add + norm, then the MLP from the HIP step's normed input
    x_mid = x + attn_out
    h2 = cap.mlp_in[i].cpu()
    assert_close(h2, rms_norm(x_mid, _w(layer.post_attention_layernorm), eps), BF16_ATOL,
                 f"layer {i} post-attention norm", rtol=BF16_RTOL)
    mlp = layer.mlp
    h2f = h2.float()
    gate = _bf(h2f @ _w(mlp.gate_proj).t())
    up = _bf(h2f @ _w(mlp.up_proj).t())
    m = _bf(swiglu(gate, up)) @ _w(mlp.down_proj).t()
    mlp_out = cap.mlp_out[i].cpu()
    assert_close(mlp_out, m, BF16_ATOL, f"layer {i} mlp out", rtol=BF16_RTOL)
    return x_mid, mlp_out


def _check_greedy(model, cfg, hidden, ids, best, x_last, pending):
    """Final norm and the greedy id against the oracle (one bf16 ulp of slack
    where two candidates' exact logits tie within rounding, as in the lm_head
    tests)."""
    hid = hidden.cpu()
    ref_h = rms_norm(x_last + pending, _w(model.model.norm), cfg.rms_norm_eps)
    assert_close(hid, ref_h.view(B, -1), BF16_ATOL, "final norm", rtol=BF16_RTOL)
    W = model.lm_head.weight.detach()
    ref_ids, _, ref_logits = oracle_argmax(hid, W)
    got = ids.view(-1).cpu()
    mism = (got != ref_ids).nonzero().view(-1).tolist()
    assert len(mism) <= 1, f"greedy ids differ in {len(mism)} rows"
    for b in mism:
        h64, w64 = hid[b].double(), W.cpu().double()
        la, lr = float(h64 @ w64[int(got[b])]), float(h64 @ w64[int(ref_ids[b])])
        assert abs(la - lr) <= BF16_RTOL * abs(lr), f"row {b}: {la} vs {lr}"
    top = ref_logits.float().gather(-1, got.view(-1, 1)).view(-1)
    assert ((best.cpu() - top).abs() <= BF16_RTOL * top.abs()).all()


def _eager_step(model, cache, ids):
    _reset(cache)
    with torch.no_grad():
        out = model.model(ids, past_key_values=cache, use_cache=True)
        hidden = out["hidden_states"][:, -1, :]
        from llm_cuda.kernels._ops import lm_head_argmax

        nxt, best = lm_head_argmax(hidden, model.lm_head.weight, return_max=True)
    torch.cuda.synchronize()
    return hidden, nxt, best


@pytest.mark.parametrize("projections", ["native", "torch"])
def test_config4_two_layers_every_block_matches_oracle(cuda, monkeypatch, projections):
    """Two full-width layers of the config-4 step (full vocabulary), every block
    of both layers and the greedy ids against the oracle; with the projections
    on the native kernel, and as torch matmuls (BASELINE config 4 as stated:
    the MLP's [gate; up] weight then kept transposed, the parameters views of
    it)."""
    import contextlib

    from llm_cuda.kernels import _ops

    cfg, model, cache, ids = _build(cuda, layers=2)
    cap = _Capture(model, monkeypatch)
    ctx = _ops.torch_projections() if projections == "torch" else contextlib.nullcontext()
    with ctx:
        hidden, nxt, best = _eager_step(model, cache, ids)
    cap.remove()
    if projections == "torch":
        mlp = model.model.layers[0].mlp
        wt = mlp._gate_up.buf
        assert mlp._gate_up.columns and wt.shape == (cfg.hidden_size, 2 * cfg.intermediate_size)
        assert mlp.up_proj.weight.data_ptr() == wt.data_ptr() + cfg.intermediate_size * 2
    assert len(cap.dec) == 2 and len(cap.attn_in) == 2 and len(cap.mlp_out) == 2
    # 32 sequences x 8 kv heads fill the 256 CUs once: the fused step runs
    assert cap.fused == 2 or torch.cuda.get_device_properties(0).multi_processor_count != 256
    x = model.model.embed_tokens.weight.detach()[ids.view(-1)].view(B, 1, -1).cpu()
    pending = None
    for i in range(2):
        x, pending = _check_layer(model, cache, cfg, cap, i, x, pending)
    _check_greedy(model, cfg, hidden, nxt, best, x, pending)


def test_config4_full_step_graph_layers_and_argmax(cuda, monkeypatch):
    """The full 32-layer config-4 step: HIP-graph replays equal the eager step
    bit for bit, the fused argmax is the argmax of the step's logits, and layers
    0 and 31 (plus the greedy ids) match the oracle."""
    cfg, model, cache, ids = _build(cuda, layers=32)
    cap = _Capture(model, monkeypatch)
    hidden, nxt, best = _eager_step(model, cache, ids)
    cap.remove()
    monkeypatch.undo()
    assert len(cap.dec) == 32

    # Layer 0 from the embedding. Layer 31 from the residual stream the HIP
    # step carried into it, rebuilt from the captured block outputs with the
    # model's own bf16 adds: x_mid_i = x_in_i + attn_i, x_in_{i+1} = x_mid_i + mlp_i.
    emb = model.model.embed_tokens.weight.detach()[ids.view(-1)].view(B, 1, -1).cpu()
    x_mid, mlp_out = _check_layer(model, cache, cfg, cap, 0, emb, None)
    for i in range(1, 31):
        x_mid, mlp_out = x_mid + mlp_out + cap.attn_out[i].cpu(), cap.mlp_out[i].cpu()
    x_mid, mlp_out = _check_layer(model, cache, cfg, cap, 31, x_mid, mlp_out)
    _check_greedy(model, cfg, hidden, nxt, best, x_mid, mlp_out)

    # graph capture and replays
    def step():
        cache.seq_lens_all.fill_(CTX)
        ids_out, _, top = model.greedy_next_token(ids, cache, return_logit=True)
        return ids_out, top

    with torch.no_grad():
        _reset(cache)
        e_ids, e_top = step()
        e_ids, e_top = e_ids.clone(), e_top.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            _reset(cache)
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        _reset(cache)
        with torch.cuda.graph(graph):
            g_ids, g_top = step()
        for r in range(3):
            _reset(cache)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(g_ids, e_ids), f"replay {r}: ids differ from the eager step"
            assert torch.equal(g_top, e_top), f"replay {r}: winning logits differ"
            # eager work between replays
            scratch = torch.randn(1024, 1024, device=cuda) @ torch.randn(1024, 1024, device=cuda)
            del scratch
            torch.cuda.synchronize()
        assert torch.equal(e_ids.view(-1), nxt.view(-1))

        # the fused argmax against torch.argmax over the step's full logits
        _reset(cache)
        full = model(input_ids=ids, past_key_values=cache, use_cache=True)["logits"][:, -1, :]
        ref_ids = torch.argmax(full, dim=-1)
        top = full.float().gather(-1, e_ids.view(-1, 1)).view(-1)
        ref_top = full.float().gather(-1, ref_ids.view(-1, 1)).view(-1)
        assert ((top - ref_top).abs() <= BF16_RTOL * ref_top.abs()).all()
        assert (e_ids.view(-1) == ref_ids).float().mean().item() >= 31 / 32
    del graph
    torch.cuda.synchronize()
