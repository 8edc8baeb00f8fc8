"""SwiGLU forward entry (reference: kernels/triton/swiglu.py:91-145,199-200).

out = silu(gate) * up computed in fp32 by the lc_swiglu_fwd HIP kernel for any
width (the reference's Triton kernel clamped its block to 4096 columns). Only
the forward pass is provided: when gate or up requires grad, the result is
recorded in the autograd graph, and a backward through it raises
RuntimeError instead of returning a wrong or missing gradient.
"""
from __future__ import annotations

import torch

from llm_cuda.kernels import _ops


def triton_swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return _ops.swiglu(gate, up)
