"""Pins the lm_head + greedy argmax oracle (oracle/lm_head.py).

Checks, each of which a plausible slip would fail:
  * brute force: per-row Python loops over exact fp64 dot products, rounding
    and a first-index scan (catches a transposed weight, a wrong tie rule);
  * the reference's op sequence on the host, torch.argmax(F.linear(h, W)) in
    fp32 (model.py:156,214): identical ids wherever the two rounded logits agree;
  * ties across the whole vocabulary go to the smallest index; NaN ranks first.
"""
import torch
import torch.nn.functional as F

from oracle.lm_head import argmax_first, lm_head_argmax, lm_head_logits


def test_brute_force_small():
    g = torch.Generator().manual_seed(3)
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        h = torch.randn(3, 7, generator=g).to(dtype)
        w = torch.randn(11, 7, generator=g).to(dtype)
        ids, best, logits = lm_head_argmax(h, w)
        for b in range(3):
            vals = []
            for v in range(11):
                acc = sum(float(h[b, k]) * float(w[v, k]) for k in range(7))
                vals.append(float(torch.tensor(acc, dtype=torch.float64).to(dtype)))
            top = max(vals)
            assert ids[b].item() == vals.index(top)
            assert best[b].item() == top
            assert torch.equal(logits[b].double(), torch.tensor(vals, dtype=torch.float64))


def test_matches_reference_op_sequence():
    """argmax(F.linear(h, W)) as the reference computes it, with fp32 logits."""
    g = torch.Generator().manual_seed(0)
    h = torch.randn(8, 256, generator=g)
    w = torch.randn(32000, 256, generator=g) * 0.02
    ids, _, _ = lm_head_argmax(h, w)
    ref = torch.argmax(F.linear(h, w), dim=-1)
    assert torch.equal(ids, ref)


def test_ties_pick_first_index_and_nan_ranks_first():
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [0.0, 0.0, 0.0, 0.0],
                      [1.0, float("nan"), 5.0, float("nan")], [-1.0, -2.0, -1.0, -3.0]])
    assert argmax_first(x).tolist() == [1, 0, 1, 0]
    assert argmax_first(x).tolist() == torch.argmax(x, dim=-1).tolist()


def test_equal_weight_rows_resolve_to_smallest_index():
    g = torch.Generator().manual_seed(1)
    h = torch.randn(4, 64, generator=g).bfloat16()
    w = torch.randn(500, 64, generator=g).bfloat16()
    ids, _, _ = lm_head_argmax(h, w)
    w2 = w.clone()
    for b in range(4):
        w2[499 - b] = w[ids[b]]  # a later copy of the winner changes nothing
    ids2, _, _ = lm_head_argmax(h, w2)
    assert torch.equal(ids, ids2)


def test_rounding_to_model_dtype_happens_before_the_comparison():
    """Two logits that differ in fp64 but round to the same bf16 tie: the smaller
    index wins, as torch.argmax on bf16 logits would pick."""
    h = torch.tensor([[1.0, 1.0]], dtype=torch.bfloat16)
    w = torch.tensor([[1.0, 0.0], [1.0, 2.0 ** -10]], dtype=torch.bfloat16)
    logits = lm_head_logits(h, w)
    assert logits[0, 0] == logits[0, 1]
    ids, _, _ = lm_head_argmax(h, w)
    assert ids.item() == 0
    ids32, _, _ = lm_head_argmax(h.float(), w.float())
    assert ids32.item() == 1
