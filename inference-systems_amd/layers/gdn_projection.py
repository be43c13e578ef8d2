"""Merged input projection of the gated-delta-net layer.

nanovllm/layers/gated_delta_net.py:60-63 applies four bias-free projections
to the same hidden states -- ``in_proj_qkv`` (2 key_dim + value_dim rows),
``in_proj_z`` (value_dim), ``in_proj_b`` and ``in_proj_a`` (one row per value
head) -- and calls them one after the other (gated_delta_net.py:192-195,
331-338).  Here their weights are rows of one W[N, K] with
N = conv_dim + value_dim + 2 * num_value_heads (8224 for Qwen3.5-0.8B:
6144 + 2048 + 16 + 16), so a decode step reads the activations once and
streams one weight matrix in one GEMM launch instead of four.

The checkpoint still holds four tensors.  ``weight_loader(param, w,
shard_id)`` with shard_id in {"qkv", "z", "b", "a"} writes each one into its
row range, applying the same tensor-parallel narrowing as the reference's
loaders (gated_delta_net.py:93-110): q, k and v are cut per rank from their
own thirds of the qkv tensor, z per rank by value_dim rows, a and b per rank
by num_value_heads rows.  ``forward`` returns the four outputs in the order
qkv, z, b, a, as views of the one GEMM result.  With one row of activations
(single-sequence decode) those views are contiguous.  With several rows a
column range is strided; the reference's batched decode hands the four
projections to gdn_decode_core, whose CUDA path takes contiguous tensors only
(nanovllm/kernels/gdn.py:186), so ``forward(x, contiguous=True)`` gives
contiguous outputs there by running the four GEMMs on the weight's row
ranges (what the reference does), not one GEMM and four copies: measured on
MI355X at M = 32 (N = 8224, K = 1024, bf16, W from HBM), one GEMM with
views 8.6 us, the four GEMMs 17.7 us, one GEMM plus four .contiguous()
copies 20.0 us.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from ..kernels import add_rmsnorm_linear
from ..kernels import linear as gemm_linear
from .linear import _tp_rank_size, divide

SHARDS = ("qkv", "z", "b", "a")


class GdnInputProjection(nn.Module):

    def __init__(self, hidden_size: int, num_key_heads: int, num_value_heads: int, key_head_dim: int,
                 value_head_dim: int):
        super().__init__()
        self.tp_rank, self.tp_size = _tp_rank_size()
        if num_value_heads % num_key_heads:
            raise ValueError("num_value_heads must be a multiple of num_key_heads")
        self.total_num_key_heads = num_key_heads
        self.total_num_value_heads = num_value_heads
        self.key_head_dim = key_head_dim
        self.value_head_dim = value_head_dim
        self.num_key_heads = divide(num_key_heads, self.tp_size)
        self.num_value_heads = divide(num_value_heads, self.tp_size)
        self.key_dim = self.num_key_heads * key_head_dim
        self.value_dim = self.num_value_heads * value_head_dim
        self.conv_dim = 2 * self.key_dim + self.value_dim
        self.output_sizes = (self.conv_dim, self.value_dim, self.num_value_heads, self.num_value_heads)
        starts = [0]
        for size in self.output_sizes[:-1]:
            starts.append(starts[-1] + size)
        self.shard_offsets = dict(zip(SHARDS, starts))
        self.shard_sizes = dict(zip(SHARDS, self.output_sizes))
        self.weight = nn.Parameter(torch.empty(sum(self.output_sizes), hidden_size))
        self.weight.weight_loader = self.weight_loader
        self.gemm_backend: Optional[str] = None   # None: NANOVLLM_GEMM_BACKEND

    def _rank_rows(self, loaded_weight: torch.Tensor, shard_id: str) -> torch.Tensor:
        """This rank's rows of one checkpoint tensor."""
        r = self.tp_rank
        if shard_id == "qkv":
            total_key = self.total_num_key_heads * self.key_head_dim
            q = loaded_weight.narrow(0, r * self.key_dim, self.key_dim)
            k = loaded_weight.narrow(0, total_key + r * self.key_dim, self.key_dim)
            v = loaded_weight.narrow(0, 2 * total_key + r * self.value_dim, self.value_dim)
            return torch.cat((q, k, v), dim=0)
        if shard_id == "z":
            return loaded_weight.narrow(0, r * self.value_dim, self.value_dim)
        return loaded_weight.narrow(0, r * self.num_value_heads, self.num_value_heads)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: str):
        if loaded_shard_id not in SHARDS:
            raise ValueError(f"unknown shard id {loaded_shard_id!r}; expected one of {SHARDS}")
        rows = self._rank_rows(loaded_weight, loaded_shard_id)
        param.data.narrow(0, self.shard_offsets[loaded_shard_id], self.shard_sizes[loaded_shard_id]).copy_(rows)

    def forward(self, x: torch.Tensor,
                contiguous: bool = False) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
        if contiguous and x.numel() // x.shape[-1] > 1:
            return tuple(gemm_linear(x, self.weight.narrow(0, self.shard_offsets[sid], self.shard_sizes[sid]), None,
                                     backend=self.gemm_backend) for sid in SHARDS)
        y = gemm_linear(x, self.weight, None, backend=self.gemm_backend)
        return y.split(self.output_sizes, dim=-1)

    def forward_add_norm(self, hidden: torch.Tensor, residual: torch.Tensor, norm):
        """``(self(norm(hidden, residual)), new residual)``: the input norm of
        a linear-attention decoder layer and the merged projection
        (nanovllm/models/qwen3_5.py:157-163).  On the HIP path the residual
        add and the norm run inside the GEMM."""
        y, new_residual = add_rmsnorm_linear(hidden, residual, norm.weight, norm.eps, self.weight,
                                             backend=self.gemm_backend)
        return y.split(self.output_sizes, dim=-1), new_residual
