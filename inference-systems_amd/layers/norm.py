"""Qwen3.5's zero-centred RMSNorm (nanovllm/layers/layernorm.py:110-142).

The checkpoint stores a zero-centred scale and the norm applies ``1 + weight``
in fp32.  With a residual, ``forward(x, residual)`` returns
(round(norm(x + residual)), round(x + residual)).  This module runs the
reference arithmetic in torch; the projections that follow a norm take it
as a prologue (``Qwen35MLP.forward_add_norm``,
``GdnInputProjection.forward_add_norm``), where on the HIP path the add and
the norm run inside the GEMM.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from ..kernels import torch_add_rmsnorm


class Qwen35RMSNorm(nn.Module):

    def __init__(self, hidden_size: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.zeros(hidden_size))

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None):
        if residual is None:
            x32 = x.float()
            normalized = x32 * torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + self.eps)
            return (normalized * (1.0 + self.weight.float())).to(x.dtype)
        return torch_add_rmsnorm(x, residual, self.weight, self.eps)
