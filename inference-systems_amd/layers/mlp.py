"""Qwen3.5 MLP with the fused gate/up projection and SiLU-and-mul.

Same submodules, weight layout and tensor-parallel sharding as the
reference's MLP (nanovllm/models/qwen3_5.py:105-118): ``gate_up_proj`` is a
MergedColumnParallelLinear over [intermediate, intermediate] rows,
``down_proj`` a RowParallelLinear.  The reference computes
``down_proj(SiluAndMul(gate_up_proj(x)))``, writing and re-reading the
[T, 2 * intermediate] projection; on the HIP path ``gate_up_proj`` and
SiluAndMul (nanovllm/layers/activation.py:8-11) are one launch of
``nanovllm::gemm_silu_mul``.  Each rank's gate_up weight is [gate rows of
the rank; up rows of the rank], exactly the layout the fused op takes.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from ..kernels import add_rmsnorm_linear, silu_mul_linear
from .linear import MergedColumnParallelLinear, RowParallelLinear
from .norm import Qwen35RMSNorm


class Qwen35MLP(nn.Module):

    def __init__(self, hidden_size: int, intermediate_size: int, hidden_act: str = "silu"):
        super().__init__()
        if hidden_act != "silu":
            raise ValueError("Qwen3.5 MLP currently supports only SiLU")
        self.gate_up_proj = MergedColumnParallelLinear(hidden_size, [intermediate_size, intermediate_size],
                                                       bias=False)
        self.down_proj = RowParallelLinear(intermediate_size, hidden_size, bias=False)
        self._gemm_backend: Optional[str] = None

    @property
    def gemm_backend(self) -> Optional[str]:
        return self._gemm_backend

    @gemm_backend.setter
    def gemm_backend(self, value: Optional[str]) -> None:
        """Backend of both projections (None: NANOVLLM_GEMM_BACKEND)."""
        self._gemm_backend = value
        self.gate_up_proj.gemm_backend = value
        self.down_proj.gemm_backend = value

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = silu_mul_linear(x, self.gate_up_proj.weight, backend=self._gemm_backend)
        return self.down_proj(h)

    def forward_add_norm(self, hidden: torch.Tensor, residual: torch.Tensor,
                         norm: Qwen35RMSNorm) -> tuple[torch.Tensor, torch.Tensor]:
        """``self(norm(hidden, residual))`` with the new residual: the
        post-attention norm and MLP of a decoder layer
        (nanovllm/models/qwen3_5.py:200-204).  On the HIP path the residual
        add, the norm, gate_up_proj and SiluAndMul are one launch."""
        h, new_residual = add_rmsnorm_linear(hidden, residual, norm.weight, norm.eps, self.gate_up_proj.weight,
                                             silu_mul=True, backend=self._gemm_backend)
        return self.down_proj(h), new_residual
