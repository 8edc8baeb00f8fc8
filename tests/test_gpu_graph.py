"""HIP-graph capture of a decode step that runs only this library's kernels
and torch matmuls: paged decode with the fused RoPE + KV append, add + RMSNorm,
SwiGLU, and the fused lm_head + greedy argmax.

The graph is replayed several times with eager work and synchronisations in
between; every replay must reproduce the eager step exactly (same ids and the
same winning logits), which is what a captured serving loop relies on (no
memset nodes, no host-side state baked into the graph).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_decode_step_graph_replays_match_eager(cuda):
    from llm_cuda.models.llama3.config import Llama3Config
    from llm_cuda.models.llama3.kv_cache import PagedKVCache
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = Llama3Config(vocab_size=3000, hidden_size=256, intermediate_size=512,
                       num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                       max_position_embeddings=512)
    torch.manual_seed(0)
    model = Llama3ForCausalLM(cfg).to(device=cuda, dtype=torch.bfloat16).eval()
    B, ctx, P = 4, 100, 16
    cache = PagedKVCache.create(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim,
                                256, P, cuda, torch.bfloat16, batch_size=B)
    g = torch.Generator(device=cuda).manual_seed(0)
    for layer in cache.layer_caches:
        layer.key_pages.normal_(generator=g)
        layer.value_pages.normal_(generator=g)
    ids = torch.randint(0, cfg.vocab_size, (B, 1), generator=g, device=cuda)

    def reset():
        cache.seq_lens_all.fill_(ctx)
        for layer in cache.layer_caches:
            layer.lengths = [ctx] * B

    def step():
        cache.seq_lens_all.fill_(ctx)
        nxt, _, best = model.greedy_next_token(ids, cache, return_logit=True)
        return nxt, best

    with torch.no_grad():
        reset()
        eager_ids, eager_best = (t.clone() for t in step())
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                reset()
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        reset()
        with torch.cuda.graph(graph):
            g_ids, g_best = step()
        for rep in range(4):
            reset()
            # unrelated eager work between replays
            junk = torch.randn(1 << 20, device=cuda).sum()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.isfinite(junk)
            assert torch.equal(g_ids, eager_ids), f"replay {rep}: ids differ"
            assert torch.equal(g_best, eager_best), f"replay {rep}: winning logits differ"


@pytest.mark.parametrize("eager_first", [True, False])
def test_ragged_decode_graph_replays_with_ticket(cuda, eager_first):
    """A ragged paged decode whose split workgroups take several rounds of the
    CUs (the longest-first order with its ticket-handed tail) captured in a HIP
    graph: with an eager call first the capture uses the per-device graph
    counters, without one it runs the static order. Every replay, with eager
    calls in between, reproduces the eager output bit for bit, and the graph
    counters are back at zero after each replay."""
    import math

    from llm_cuda.kernels import _ops
    from llm_cuda.kernels.triton.decode_attention import paged_decode_attention

    _ops._COUNTERS.pop(("paged_decode", "cuda", cuda.index, "graphs"), None)
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, D, P = 64, 32, 8, 128, 64
    lens = torch.randint(512, 8193, (B,), generator=g)
    maxp = math.ceil(int(lens.max()) / P)
    N = B * maxp
    bt = torch.randperm(N, generator=g).to(torch.int32).view(B, maxp).to(cuda)
    kp = torch.randn(N, Hkv, P, D, generator=g).to(torch.bfloat16).to(cuda)
    vp = torch.randn(N, Hkv, P, D, generator=g).to(torch.bfloat16).to(cuda)
    q = torch.randn(B, Hq, 1, D, generator=g).to(torch.bfloat16).to(cuda)
    sl = lens.to(torch.int32).to(cuda)

    def run():
        return paged_decode_attention(q, kp, vp, bt, sl, return_lse=True)

    ref_out, ref_lse = run()
    ref_out, ref_lse = ref_out.clone(), ref_lse.clone()
    if not eager_first:
        _ops._COUNTERS.pop(("paged_decode", "cuda", cuda.index, "graphs"), None)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            g_out, g_lse = run()
    torch.cuda.current_stream().wait_stream(side)
    key = ("paged_decode", "cuda", cuda.index, "graphs")
    assert (key in _ops._COUNTERS) == eager_first
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_out, ref_out), f"replay {rep}: output differs from eager"
        assert torch.equal(g_lse, ref_lse), f"replay {rep}: lse differs from eager"
        if eager_first:
            assert int(_ops._COUNTERS[key].abs().sum()) == 0
        out, lse = run()  # eager work between replays
        assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)


@pytest.mark.parametrize("dtype,batch,kv_heads,new", [
    (torch.float32, 2, 2, 5),     # fp32 (config 1's dtype): RoPE + append, then split-K decode
    (torch.bfloat16, 32, 8, 6),   # 256 (sequence, kv head) units: the fused decode step
    (torch.bfloat16, 3, 4, 7),    # split-K decode in bf16
    (torch.bfloat16, 3, 4, 2),    # two eager steps, nothing to replay
    (torch.bfloat16, 3, 4, 1),
])
def test_generate_with_graph_equals_eager(cuda, dtype, batch, kv_heads, new):
    """generate(use_graph=True): the prompt and the first decode step eager,
    the rest replays of one captured step that reads its positions from the
    cache's device-side lengths. The ids equal the eager loop's (the same
    kernels on the same inputs), and use_graph without the paged cache raises."""
    from llm_cuda.models.llama3.config import Llama3Config
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    torch.manual_seed(11)
    cfg = Llama3Config(vocab_size=2000, hidden_size=512, intermediate_size=1024,
                       num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=kv_heads,
                       max_position_embeddings=512)
    model = Llama3ForCausalLM(cfg).to(device=cuda, dtype=dtype).eval()
    ids = torch.randint(0, cfg.vocab_size, (batch, 9), device=cuda)
    eager = model.generate(ids, max_new_tokens=new, use_paged_kv=True)
    graphed = model.generate(ids, max_new_tokens=new, use_paged_kv=True, use_graph=True)
    torch.cuda.synchronize()
    assert graphed.shape == (batch, 9 + new)
    assert torch.equal(graphed, eager)
    with pytest.raises(ValueError):
        model.generate(ids, max_new_tokens=2, use_graph=True)
