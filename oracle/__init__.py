"""CPU oracle for the Llama-3 attention path — TEST INFRASTRUCTURE ONLY.

A plain restatement of the reference's algorithms (calvin-fei/llm-cuda,
src/llm_cuda/...), each function citing the reference file:line it follows.
Floating-point functions compute in torch fp32 on the host from the same
(possibly bf16) inputs; page-table indexing is numpy integer arithmetic.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline. The
product (llm-cuda_amd/llm_cuda) never imports it and has no CPU path.

How each function is pinned (tests/test_oracle_*.py):
  attention.causal_attention  brute-force fp64 loops, row-0 / equal-key /
                              S=1 closed forms, lse invariant, q_offset
                              equivalence to the last rows of a longer prompt
  decode.decode_attention     == last row of causal_attention; kv_len=1 -> v;
                              fp64 loop of tests/test_triton_decode_attention.py:26-58
  decode.gather_pages         identity table == the reference's get_kv concat
                              semantics (kv_cache.py:65-83); random
                              permutation == element-wise brute force
  decode.merge_splits         split-count invariance, lse = logsumexp(split lses)
  rope.*                      complex-multiplication formulation, position 0 =
                              identity, norm preservation, half-table equality
  norm.rms_norm               constant-row closed form, fp64 formula
  swiglu.swiglu               g = 0 -> 0, large g -> g*u, fp64 formula
  model.*                     paged/cached decode == full recompute; module
                              order reproduces the reference's seeded weights
"""
