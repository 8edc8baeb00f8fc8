"""Golden values written by the reference implementation itself
(tests/golden/make_reference_model_fixture.py): a seed-0 tiny Llama-3.

CPU: this package's Llama3ForCausalLM built under the same seed reproduces
the reference's weights tensor by tensor (module construction order and the
_init_weights traversal match) and the same prompt draw; the oracle's fp32
forward reproduces the reference's logits and greedy ids.
GPU: the HIP model reproduces them too, with and without the paged cache.
"""
import json
from pathlib import Path

import pytest
import torch

import oracle.model as omodel

FIX = json.loads((Path(__file__).parent / "golden" / "reference_tiny_llama3.json").read_text())


def _build():
    from llm_cuda.models.llama3.config import Llama3Config
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = Llama3Config(**FIX["config"])
    torch.manual_seed(FIX["seed"])
    model = Llama3ForCausalLM(cfg).eval()
    prompt = torch.randint(0, cfg.vocab_size, (2, 12))
    return cfg, model, prompt


def _ref_logits():
    return torch.tensor(FIX["logits"]).view(*FIX["logits_shape"])


def test_seeded_weights_and_prompt_match_reference():
    cfg, model, prompt = _build()
    assert prompt.tolist() == FIX["prompt"]
    sd = model.state_dict()
    assert set(sd) == set(FIX["weight_checksums"])
    for name, (s1, s2, head) in FIX["weight_checksums"].items():
        t = sd[name].double()
        assert float(t.sum()) == s1 and float(t.pow(2).sum()) == s2, name
        assert [float(x) for x in sd[name].flatten()[:4]] == head, name


def test_oracle_model_matches_reference_logits_and_generate():
    cfg, model, prompt = _build()
    logits = omodel.forward(model.state_dict(), cfg, prompt)
    assert (logits - _ref_logits()).abs().max().item() < 1e-5
    ids, _ = omodel.greedy(model.state_dict(), cfg, prompt, 6)
    assert ids.tolist() == FIX["generate_ids"]


@pytest.mark.gpu
@pytest.mark.parametrize("paged", [False, True])
def test_hip_model_matches_reference(cuda, paged):
    cfg, model, prompt = _build()
    model = model.to(cuda)
    with torch.no_grad():
        logits = model(input_ids=prompt.to(cuda))["logits"].cpu()
    assert (logits - _ref_logits()).abs().max().item() < 1e-4
    ids = model.generate(prompt.to(cuda), max_new_tokens=6, use_paged_kv=paged, page_size=4)
    assert ids.cpu().tolist() == FIX["generate_ids"]
