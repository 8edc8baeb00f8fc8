"""Write tests/golden/reference_tiny_llama3.json from the reference implementation.

Run in the build container only (the reference is not present on GPU boxes):
    python tests/golden/make_reference_model_fixture.py /root/reference/src

It imports calvin-fei/llm-cuda's Llama3ForCausalLM on the CPU (its torch
fallback paths), builds a small model under torch.manual_seed(0) and records:
per-tensor weight checksums (to pin module construction order and the
_init_weights traversal, models/llama3/model.py:110-139), the prompt ids,
the full-forward logits and the non-paged greedy generate() ids
(model.py:178-218). These are the only values of the path that no closed
form or invariant pins: they depend on the reference's RNG consumption order.
"""
import json
import sys
from pathlib import Path

import torch

CONFIG = dict(vocab_size=512, hidden_size=64, intermediate_size=172, num_hidden_layers=2,
              num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=128)
OUT = Path(__file__).resolve().parent / "reference_tiny_llama3.json"


def main(src: str) -> None:
    sys.path.insert(0, src)
    from llm_cuda.models.llama3.config import Llama3Config
    from llm_cuda.models.llama3.model import Llama3ForCausalLM

    cfg = Llama3Config(**CONFIG)
    torch.manual_seed(0)
    model = Llama3ForCausalLM(cfg).eval()
    prompt = torch.randint(0, cfg.vocab_size, (2, 12))
    with torch.no_grad():
        logits = model(input_ids=prompt)["logits"]
    gen = model.generate(prompt, max_new_tokens=6)
    sums = {n: [float(t.double().sum()), float(t.double().pow(2).sum()),
                [float(x) for x in t.flatten()[:4]]]
            for n, t in model.state_dict().items()}
    OUT.write_text(json.dumps({
        "config": CONFIG, "seed": 0, "prompt": prompt.tolist(),
        "weight_checksums": sums,
        "logits": [round(float(x), 7) for x in logits.flatten()],
        "logits_shape": list(logits.shape),
        "generate_ids": gen.tolist(),
    }))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
