"""Concatenated projection weights for inference (one GEMM instead of several).

`FusedLinearWeights(a, b, ...)` builds W = cat(a.weight, b.weight, ...) along
the output dimension the first time it is used, and re-points each Linear's
parameter at its row block of W, so the fused matrix costs no extra memory
and state-dict loads (which copy into the parameters in place) keep it
current. If a parameter is later replaced or moved (`.to()`, a new
`nn.Parameter`), the aliasing check fails and W is rebuilt. Callers use it
only when no autograd graph is being recorded; training keeps the separate
Linear calls.

`weight(columns=True)` stores the same matrix transposed, [K, sum N]
contiguous, with each parameter a transposed column block of it (a [N, K]
view with strides (1, sum N)): for a torch matmul at decode-step rows
hipBLASLt runs x @ W^T faster from that layout for the MLP's [gate; up]
weight. The parameters keep their shapes and values, and asking for the
other layout rebuilds the buffer (one copy).
"""
from __future__ import annotations

import torch
import torch.nn as nn


class FusedLinearWeights:
    def __init__(self, *linears: nn.Linear):
        if not linears or any(lin.bias is not None for lin in linears):
            raise ValueError("fused weights need bias-free Linear layers")
        self.linears = linears
        self.buf: torch.Tensor | None = None
        self.columns = False

    @staticmethod
    def usable(*linears: nn.Linear) -> bool:
        return not (torch.is_grad_enabled() and any(l.weight.requires_grad for l in linears))

    def _aliased(self, columns: bool) -> bool:
        buf = self.buf
        if buf is None or columns != self.columns:
            return False
        if columns:
            K, total = buf.shape
            off = 0
            for lin in self.linears:
                w = lin.weight
                if (w.device != buf.device or w.dtype != buf.dtype or w.dim() != 2
                        or w.shape[1] != K or w.stride() != (1, total)
                        or w.data_ptr() != buf.data_ptr() + off * buf.element_size()):
                    return False
                off += w.shape[0]
            return off == total
        cols = buf.shape[1]
        step = buf.element_size() * cols
        off = 0
        for lin in self.linears:
            w = lin.weight
            if (w.device != buf.device or w.dtype != buf.dtype or w.dim() != 2
                    or w.shape[1] != cols or not w.is_contiguous()
                    or w.data_ptr() != buf.data_ptr() + off * step):
                return False
            off += w.shape[0]
        return off == buf.shape[0]

    def weight(self, columns: bool = False) -> torch.Tensor:
        """W = cat(weights) [sum N, K], or with columns=True W^T stored
        contiguously [K, sum N]."""
        if not self._aliased(columns):
            with torch.no_grad():
                ws = [lin.weight.detach() for lin in self.linears]
                if columns:
                    buf = torch.cat([w.t() for w in ws], dim=1).contiguous()
                else:
                    buf = torch.cat(ws, dim=0)
                off = 0
                for lin in self.linears:
                    n = lin.weight.shape[0]
                    lin.weight.data = buf[:, off:off + n].t() if columns else buf[off:off + n]
                    off += n
            self.buf = buf
            self.columns = columns
        return self.buf

    def sizes(self) -> list[int]:
        return [lin.weight.shape[0] for lin in self.linears]
