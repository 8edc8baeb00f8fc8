"""Llama-3 MLP (reference: models/llama3/mlp.py:1-43): down(silu(gate(x)) * up(x)).

The projections are torch matmuls (hipBLASLt); the SwiGLU between them is the
HIP kernel.
"""
import torch
import torch.nn as nn

from llm_cuda.kernels.triton.swiglu import triton_swiglu

from .config import Llama3Config


class Llama3MLP(nn.Module):
    def __init__(self, config: Llama3Config):
        super().__init__()
        if config.tensor_parallel_size > 1:
            raise NotImplementedError("tensor parallelism is not part of this build")
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(triton_swiglu(self.gate_proj(x), self.up_proj(x)))
