"""RMSNorm module (reference: models/llama3/norm.py:1-33).

`use_triton` / `use_cuda_extension` are accepted for signature compatibility;
there is one implementation, the HIP kernel.
"""
import torch
import torch.nn as nn

from llm_cuda.kernels.triton.rmsnorm import triton_rms_norm


class RMSNorm(nn.Module):
    def __init__(
        self,
        hidden_size: int,
        eps: float = 1e-5,
        use_triton: bool = True,
        use_cuda_extension: bool = True,
    ):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.eps = eps
        self.use_triton = use_triton
        self.use_cuda_extension = use_cuda_extension

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return triton_rms_norm(x, self.weight, self.eps)
