"""GPU model-level parity (the harness of benchmark configs 1 and 4).

* Config 1 (tiny Llama-3, fp32, dim 256, 4 layers, 8/2 heads, FFN 688,
  vocab 32000, batch 2, prompt 64, 16 greedy steps, paged KV with P 64) runs
  on the HIP kernels and is compared with the oracle's full-recompute greedy
  decode on the same weights: identical ids, logits within 1e-4.
* The reference's own model tests (test_llama3_shapes.py:8-198): shapes,
  tuple-cache decode == full forward, paged decode == full forward.
* A reduced-depth bf16 model at the 8B layer shape: paged decode logits ==
  full-forward logits.
"""
import pytest
import torch

import oracle.model as omodel

pytestmark = pytest.mark.gpu


def _small_config(**kw):
    from llm_cuda.models.llama3.config import Llama3Config

    base = dict(vocab_size=1024, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                num_attention_heads=8, num_key_value_heads=4, max_position_embeddings=256)
    base.update(kw)
    return Llama3Config(**base)


def test_forward_shapes_and_loss(cuda):
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    torch.manual_seed(0)
    cfg = _small_config()
    model = Llama3ForCausalLM(cfg).to(cuda)
    ids = torch.randint(0, cfg.vocab_size, (2, 16), device=cuda)
    out = model(input_ids=ids, labels=ids)
    assert out["logits"].shape == (2, 16, cfg.vocab_size)
    assert out["loss"].dim() == 0 and torch.isfinite(out["loss"])


def test_full_forward_matches_oracle(cuda):
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    torch.manual_seed(123)
    cfg = _small_config()
    model = Llama3ForCausalLM(cfg).eval()
    ids = torch.randint(0, cfg.vocab_size, (2, 12))
    ref = omodel.forward(model.state_dict(), cfg, ids)
    model = model.to(cuda)
    with torch.no_grad():
        out = model(input_ids=ids.to(cuda))["logits"]
    assert (out.cpu() - ref).abs().max().item() < 1e-4


def test_tuple_cache_decode_parity(cuda):
    """test_llama3_shapes.py:47-88 on the GPU."""
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    torch.manual_seed(123)
    cfg = _small_config()
    model = Llama3ForCausalLM(cfg).to(cuda).eval()
    ids = torch.randint(0, cfg.vocab_size, (1, 12), device=cuda)
    with torch.no_grad():
        full = model(input_ids=ids)["logits"]
        past = model(input_ids=ids[:, :8], use_cache=True)["past_key_values"]
        steps = []
        for i in range(8, 12):
            o = model(input_ids=ids[:, i:i + 1], past_key_values=past, use_cache=True)
            past = o["past_key_values"]
            steps.append(o["logits"])
    assert torch.allclose(torch.cat(steps, 1), full[:, 8:], atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("batch", [1, 3])
def test_paged_decode_parity(cuda, batch):
    """test_llama3_shapes.py:152-198 (page_size 4), plus batch > 1."""
    from llm_cuda.models.llama3.kv_cache import PagedKVCache
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    torch.manual_seed(126)
    cfg = _small_config()
    model = Llama3ForCausalLM(cfg).to(cuda).eval()
    ids = torch.randint(0, cfg.vocab_size, (batch, 12), device=cuda)
    cache = PagedKVCache.create(num_layers=cfg.num_hidden_layers, num_kv_heads=cfg.num_key_value_heads,
                                head_dim=cfg.head_dim, max_seq_len=32, page_size=4, device=cuda,
                                dtype=torch.float32, batch_size=batch)
    with torch.no_grad():
        full = model(input_ids=ids)["logits"]
        model(input_ids=ids[:, :8], past_key_values=cache, use_cache=True)
        steps = [model(input_ids=ids[:, i:i + 1], past_key_values=cache, use_cache=True)["logits"]
                 for i in range(8, 12)]
    assert torch.allclose(torch.cat(steps, 1), full[:, 8:], atol=1e-5, rtol=1e-5)


def test_chunked_prefill_through_paged_cache(cuda):
    """A prompt fed in two chunks (second chunk attends to the cached first)."""
    from llm_cuda.models.llama3.kv_cache import PagedKVCache
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    torch.manual_seed(127)
    cfg = _small_config()
    model = Llama3ForCausalLM(cfg).to(cuda).eval()
    ids = torch.randint(0, cfg.vocab_size, (2, 20), device=cuda)
    cache = PagedKVCache.create(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, 32, 8,
                                cuda, torch.float32, batch_size=2)
    with torch.no_grad():
        full = model(input_ids=ids)["logits"]
        model(input_ids=ids[:, :11], past_key_values=cache, use_cache=True)
        tail = model(input_ids=ids[:, 11:], past_key_values=cache, use_cache=True)["logits"]
    assert torch.allclose(tail, full[:, 11:], atol=1e-5, rtol=1e-5)


def test_config1_tiny_llama_greedy_matches_oracle(cuda):
    """Benchmark config 1 (tiny Llama-3): seed 0, fp32, batch 2, prompt 64, 16 greedy steps, paged P 64."""
    from llm_cuda.models.llama3.config import Llama3Config
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = Llama3Config(vocab_size=32000, hidden_size=256, intermediate_size=688, num_hidden_layers=4,
                       num_attention_heads=8, num_key_value_heads=2)
    torch.manual_seed(0)
    model = Llama3ForCausalLM(cfg).eval()
    prompt = torch.randint(0, cfg.vocab_size, (2, 64))
    ref_ids, ref_logits = omodel.greedy(model.state_dict(), cfg, prompt, 16)
    model = model.to(cuda)
    ids = model.generate(prompt.to(cuda), max_new_tokens=16, use_paged_kv=True, page_size=64)
    assert torch.equal(ids.cpu(), ref_ids)
    # per-step logits of the paged run, re-derived by a full forward on the GPU
    with torch.no_grad():
        logits = model(input_ids=ids[:, :-1])["logits"][:, 63:, :]
    assert (logits.transpose(0, 1).cpu() - ref_logits).abs().max().item() < 1e-4


def test_bf16_8b_layer_shape_paged_vs_full(cuda):
    """Two layers at the Llama-3-8B layer shape in bf16: paged decode logits match
    the full forward (bf16 tolerance, relative to the logit scale)."""
    from llm_cuda.models.llama3.config import Llama3Config
    from llm_cuda.models.llama3.kv_cache import PagedKVCache
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = Llama3Config(vocab_size=2048, hidden_size=4096, intermediate_size=14336, num_hidden_layers=2,
                       num_attention_heads=32, num_key_value_heads=8)
    torch.manual_seed(1)
    model = Llama3ForCausalLM(cfg).to(device=cuda, dtype=torch.bfloat16).eval()
    ids = torch.randint(0, cfg.vocab_size, (4, 70), device=cuda)
    cache = PagedKVCache.create(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, 128, 64,
                                cuda, torch.bfloat16, batch_size=4)
    with torch.no_grad():
        full = model(input_ids=ids)["logits"].float()
        model(input_ids=ids[:, :66], past_key_values=cache, use_cache=True)
        steps = [model(input_ids=ids[:, i:i + 1], past_key_values=cache, use_cache=True)["logits"]
                 for i in range(66, 70)]
    got = torch.cat(steps, 1).float()
    scale = full[:, 66:].abs().max().item()
    assert (got - full[:, 66:]).abs().max().item() <= 3e-2 * max(1.0, scale)


def test_decode_step_partial_sums_are_bit_exact(cuda, monkeypatch):
    """At a bf16 decode step o_proj and down_proj leave their split-K sums to
    the add + RMSNorm after them (fp32 partials): the step's hidden states and
    logits equal, bit for bit, the same step with both projections summing in
    their own kernel."""
    from llm_cuda.kernels import _ops
    from llm_cuda.models.llama3.kv_cache import PagedKVCache
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = _small_config(hidden_size=512, intermediate_size=1536, num_hidden_layers=3,
                        num_attention_heads=8, num_key_value_heads=2, vocab_size=4096)
    torch.manual_seed(3)
    model = Llama3ForCausalLM(cfg).to(device=cuda, dtype=torch.bfloat16).eval()
    B = 6
    ids = torch.randint(0, cfg.vocab_size, (B, 40), device=cuda)
    calls = {"partials": 0}
    orig = _ops.decode_linear_partials

    def counting(*a, **k):
        calls["partials"] += 1
        return orig(*a, **k)

    monkeypatch.setattr(_ops, "decode_linear_partials", counting)

    def run():
        cache = PagedKVCache.create(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                                    64, 16, cuda, torch.bfloat16, batch_size=B)
        with torch.no_grad():
            model(input_ids=ids[:, :37], past_key_values=cache, use_cache=True)
            return [model(input_ids=ids[:, i:i + 1], past_key_values=cache,
                          use_cache=True)["logits"] for i in range(37, 40)]

    deferred = run()
    assert calls["partials"] == 3 * 2 * cfg.num_hidden_layers  # o and down, every layer, 3 steps
    monkeypatch.setattr(_ops, "decode_linear_partials_applies", lambda x, w: False)
    summed = run()
    for a, b in zip(deferred, summed):
        assert torch.equal(a, b)


def test_fused_projections_match_separate(cuda):
    """Inference runs q/k/v and gate/up as one GEMM each against the concatenated
    weights; with autograd recording, the separate Linear calls run. Both give
    the same logits (fp32, GEMM reassociation only), and the parameters alias
    the fused buffers afterwards."""
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    torch.manual_seed(7)
    cfg = _small_config()
    model = Llama3ForCausalLM(cfg).to(cuda).eval()
    ids = torch.randint(0, cfg.vocab_size, (2, 9), device=cuda)
    separate = model(input_ids=ids)["logits"].detach()
    with torch.no_grad():
        fused = model(input_ids=ids)["logits"]
    assert (fused - separate).abs().max().item() < 1e-4
    attn, mlp = model.model.layers[0].self_attn, model.model.layers[0].mlp
    buf = attn._qkv.buf
    assert buf is not None and attn.q_proj.weight.data_ptr() == buf.data_ptr()
    assert mlp.up_proj.weight.data_ptr() == mlp._gate_up.buf.data_ptr() + \
        mlp.gate_proj.weight.numel() * mlp.gate_proj.weight.element_size()
    # a state-dict load writes through the aliases into the fused buffers
    sd = {k: torch.randn_like(v) for k, v in model.state_dict().items()}
    model.load_state_dict(sd)
    with torch.no_grad():
        after = model(input_ids=ids)["logits"]
    ref = Llama3ForCausalLM(cfg).to(cuda).eval()
    ref.load_state_dict(sd)
    assert (after - ref(input_ids=ids)["logits"].detach()).abs().max().item() < 1e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_table_cache_is_bit_exact(cuda, dtype):
    """Slices of the cached all-positions table equal the per-call tables of
    rotary.build_rope_cache bit for bit, across a cache growth."""
    from llm_cuda.models.llama3.attention import Llama3Attention
    from llm_cuda.models.llama3.rotary import build_rope_cache

    cfg = _small_config(max_position_embeddings=4096)
    attn = Llama3Attention(cfg).to(device=cuda, dtype=dtype)
    for past, n in [(0, 7), (5, 1), (255, 3), (300, 1), (1000, 40)]:
        cos, sin = attn._rope_tables(past, n, torch.device(cuda), dtype)
        rc, rs = build_rope_cache(n, cfg.head_dim, cfg.rope_theta, torch.device(cuda), dtype,
                                  position_offset=past, inv_freq=attn.inv_freq)
        assert torch.equal(cos, rc) and torch.equal(sin, rs)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_greedy_next_token_equals_argmax_of_forward_logits(cuda, dtype):
    """The fused lm_head + argmax (greedy_next_token) picks the argmax of the
    forward's last-position logits (reference model.py:156,214), in bf16 and fp32."""
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    torch.manual_seed(5)
    cfg = _small_config(hidden_size=256, vocab_size=5000)
    model = Llama3ForCausalLM(cfg).to(device=cuda, dtype=dtype).eval()
    ids = torch.randint(0, cfg.vocab_size, (3, 10), device=cuda)
    with torch.no_grad():
        logits = model(input_ids=ids)["logits"][:, -1, :]
        nxt, cache, best = model.greedy_next_token(ids, None, return_logit=True)
    assert nxt.shape == (3, 1) and nxt.dtype == torch.int64 and cache is not None
    ref = torch.argmax(logits, dim=-1)
    for b in range(3):
        a, r = int(nxt[b, 0]), int(ref[b])
        # equal, or a tie within the logits' rounding
        assert a == r or abs(float(logits[b, a]) - float(logits[b, r])) <= 2 ** -7 * abs(float(logits[b, r]))
        assert abs(float(best[b]) - float(logits[b, a])) <= 2 ** -7 * abs(float(logits[b, a])) + 1e-6
