"""Llama-3 MLP (reference: models/llama3/mlp.py:1-43): down(silu(gate(x)) * up(x)).

The projections are torch matmuls (hipBLASLt); the SwiGLU between them is the
HIP kernel. For inference, gate and up come out of one GEMM against the
concatenated weight and SwiGLU reads the two halves of its output in place.
Inside `_ops.torch_projections()` that weight is kept transposed, [K, 2N]
(the parameters are views of it): at the 8B decode step hipBLASLt's x @ W^T
takes 44 us from that layout against 52-55 us from [2N, K].
At a decode step (at most 32 rows, bf16/f16) gate, up and the SwiGLU are one
native launch instead (`decode_linear(swiglu=True)`): the [gate; up] weight is
streamed once and only the SwiGLU output is written, with the same roundings.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from llm_cuda.kernels import _ops
from llm_cuda.kernels.triton.swiglu import triton_swiglu

from .config import Llama3Config
from .fused import FusedLinearWeights


class Llama3MLP(nn.Module):
    def __init__(self, config: Llama3Config):
        super().__init__()
        if config.tensor_parallel_size > 1:
            raise NotImplementedError("tensor parallelism is not part of this build")
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)
        self._gate_up = FusedLinearWeights(self.gate_proj, self.up_proj)

    def forward(self, x: torch.Tensor, partial_out: bool = False) -> torch.Tensor:
        """The reference's forward (mlp.py:39-43). partial_out (an extension,
        default off): at a decode step whose down_proj runs on the native
        projection kernel, return its output as an `_ops.PartialSum` (split-K
        partials) for `add_rms_norm` to add up."""
        if FusedLinearWeights.usable(self.gate_proj, self.up_proj):
            n = self.gate_proj.weight.shape[0]
            if not _ops.native_projections():
                gu = torch.matmul(x, self._gate_up.weight(columns=True))
                return self.down_proj(triton_swiglu(gu[..., :n], gu[..., n:]))
            w = self._gate_up.weight()
            if _ops.decode_linear_applies(x, w, swiglu=True):
                h = _ops.decode_linear(x, w, swiglu=True)
                wd = self.down_proj.weight
                if partial_out and _ops.decode_linear_partials_applies(h, wd):
                    return _ops.decode_linear_partials(h, wd)
                if _ops.decode_linear_applies(h, wd):
                    return _ops.decode_linear(h, wd)
                return self.down_proj(h)
            gu = F.linear(x, w)
            return self.down_proj(triton_swiglu(gu[..., :n], gu[..., n:]))
        return self.down_proj(triton_swiglu(self.gate_proj(x), self.up_proj(x)))
