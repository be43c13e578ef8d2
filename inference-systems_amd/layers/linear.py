"""nano-vLLM linear layers with the MI355X GEMM as their matmul.

Same classes, constructor arguments, weight layout ([out, in] = W[N, K]) and
tensor-parallel sharding as nanovllm/layers/linear.py:12-156 and the LM head
of nanovllm/layers/embed_head.py:45-66; the one change is the call that
computes ``x @ W^T``: ``F.linear`` (linear.py:51, 73, 153; embed_head.py:61)
becomes ``kernels.gemm.linear``, which routes to the ``nanovllm::gemm`` op.

Routing is opt-in per process with ``NANOVLLM_GEMM_BACKEND`` = ``torch``
(default, F.linear), ``hip`` or ``auto`` -- the module-level gating pattern
of nanovllm/layers/layernorm.py:17-20 -- or per module with the
``gemm_backend`` attribute.  The tensor-parallel collectives are unchanged
(one GPU here: tp_size is 1 unless a process group says otherwise).
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.distributed as dist
from torch import nn

from ..kernels import gated_linear, gemm_sample, greedy_linear, sample_contract_reason, sample_linear, torch_sampler
from ..kernels import linear as gemm_linear
from ..kernels import validate_gemm_backend
from ..kernels.gemm import default_backend


def divide(numerator: int, denominator: int) -> int:
    assert numerator % denominator == 0
    return numerator // denominator


def _tp_rank_size() -> tuple[int, int]:
    """(rank, world size) of the default process group; (0, 1) without one.

    The reference calls dist.get_rank() unconditionally (linear.py:23-24);
    a single-GPU process without a group is treated as tp_size 1."""
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank(), dist.get_world_size()
    return 0, 1


class LinearBase(nn.Module):

    def __init__(self, input_size: int, output_size: int, bias: bool = False, tp_dim: Optional[int] = None):
        super().__init__()
        self.tp_dim = tp_dim
        self.tp_rank, self.tp_size = _tp_rank_size()
        self.weight = nn.Parameter(torch.empty(output_size, input_size))
        self.weight.weight_loader = self.weight_loader
        if bias:
            self.bias = nn.Parameter(torch.empty(output_size))
            self.bias.weight_loader = self.weight_loader
        else:
            self.register_parameter("bias", None)
        self.gemm_backend: Optional[str] = None   # None: NANOVLLM_GEMM_BACKEND

    def matmul(self, x: torch.Tensor, bias: Optional[torch.Tensor]) -> torch.Tensor:
        return gemm_linear(x, self.weight, bias, backend=self.gemm_backend)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError


class ReplicatedLinear(LinearBase):

    def __init__(self, input_size: int, output_size: int, bias: bool = False):
        super().__init__(input_size, output_size, bias)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param.data.copy_(loaded_weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.matmul(x, self.bias)


class ColumnParallelLinear(LinearBase):

    def __init__(self, input_size: int, output_size: int, bias: bool = False):
        _, tp_size = _tp_rank_size()
        super().__init__(input_size, divide(output_size, tp_size), bias, 0)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param_data = param.data
        shard_size = param_data.size(self.tp_dim)
        start_idx = self.tp_rank * shard_size
        param_data.copy_(loaded_weight.narrow(self.tp_dim, start_idx, shard_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.matmul(x, self.bias)


class MergedColumnParallelLinear(ColumnParallelLinear):

    def __init__(self, input_size: int, output_sizes: list[int], bias: bool = False):
        self.output_sizes = output_sizes
        super().__init__(input_size, sum(output_sizes), bias)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: int):
        param_data = param.data
        shard_offset = sum(self.output_sizes[:loaded_shard_id]) // self.tp_size
        shard_size = self.output_sizes[loaded_shard_id] // self.tp_size
        param_data = param_data.narrow(self.tp_dim, shard_offset, shard_size)
        param_data.copy_(loaded_weight.chunk(self.tp_size, self.tp_dim)[self.tp_rank])


class QKVParallelLinear(ColumnParallelLinear):

    def __init__(self, hidden_size: int, head_size: int, total_num_heads: int,
                 total_num_kv_heads: Optional[int] = None, bias: bool = False):
        _, tp_size = _tp_rank_size()
        total_num_kv_heads = total_num_kv_heads or total_num_heads
        self.head_size = head_size
        self.num_heads = divide(total_num_heads, tp_size)
        self.num_kv_heads = divide(total_num_kv_heads, tp_size)
        output_size = (total_num_heads + 2 * total_num_kv_heads) * self.head_size
        super().__init__(hidden_size, output_size, bias)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: str):
        param_data = param.data
        assert loaded_shard_id in ["q", "k", "v"]
        if loaded_shard_id == "q":
            shard_size = self.num_heads * self.head_size
            shard_offset = 0
        elif loaded_shard_id == "k":
            shard_size = self.num_kv_heads * self.head_size
            shard_offset = self.num_heads * self.head_size
        else:
            shard_size = self.num_kv_heads * self.head_size
            shard_offset = self.num_heads * self.head_size + self.num_kv_heads * self.head_size
        param_data = param_data.narrow(self.tp_dim, shard_offset, shard_size)
        param_data.copy_(loaded_weight.chunk(self.tp_size, self.tp_dim)[self.tp_rank])


class RowParallelLinear(LinearBase):

    def __init__(self, input_size: int, output_size: int, bias: bool = False):
        _, tp_size = _tp_rank_size()
        super().__init__(divide(input_size, tp_size), output_size, bias, 1)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param_data = param.data
        if param_data.ndim == 1:
            param_data.copy_(loaded_weight)
            return
        shard_size = param_data.size(self.tp_dim)
        start_idx = self.tp_rank * shard_size
        param_data.copy_(loaded_weight.narrow(self.tp_dim, start_idx, shard_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self.matmul(x, self.bias if self.tp_rank == 0 else None)
        if self.tp_size > 1:
            dist.all_reduce(y)
        return y

    def forward_gated(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        """``self(x * sigmoid(gate))``: the output gate of Qwen3.5 gated
        attention before o_proj (nanovllm/models/qwen3_5.py:95-96).  ``x`` is
        this rank's heads [M, heads, head_dim] (or [M, K]) and ``gate`` the
        matching view of q_proj's output; on the HIP path the gate is applied
        in front of the GEMM."""
        y = gated_linear(x, gate, self.weight, backend=self.gemm_backend)
        if self.bias is not None and self.tp_rank == 0:
            y = y + self.bias.to(y.dtype)
        if self.tp_size > 1:
            dist.all_reduce(y)
        return y


class ParallelLMHead(nn.Module):
    """Tied / vocab-parallel LM head (embed_head.py:45-66).

    The reference selects the last token of each sequence from the forward
    context in prefill (embed_head.py:57-60); here the caller passes
    ``last_indices`` (or None in decode).  ``logits_dtype`` None (the
    default) keeps the reference's semantics on every backend: the logits
    come out in the model dtype, as ``F.linear`` returns them
    (embed_head.py:61), and the greedy and sampled heads rank those rounded
    values (Sampler takes ``logits.float()``, sampler.py:15), so the tokens
    are the reference's.  ``logits_dtype = torch.float32`` opts into fp32
    logits written by the GEMM directly and fp32 ranking."""

    def __init__(self, num_embeddings: int, embedding_dim: int, bias: bool = False):
        super().__init__()
        assert not bias
        self.tp_rank, self.tp_size = _tp_rank_size()
        self.num_embeddings = num_embeddings
        self.num_embeddings_per_partition = divide(num_embeddings, self.tp_size)
        self.vocab_start_idx = self.num_embeddings_per_partition * self.tp_rank
        self.vocab_end_idx = self.vocab_start_idx + self.num_embeddings_per_partition
        self.weight = nn.Parameter(torch.empty(self.num_embeddings_per_partition, embedding_dim))
        self.weight.weight_loader = self.weight_loader
        self.gemm_backend: Optional[str] = None
        self.logits_dtype: Optional[torch.dtype] = None   # None: the model dtype (the reference's)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param_data = param.data
        shard_size = param_data.size(0)
        start_idx = self.tp_rank * shard_size
        param_data.copy_(loaded_weight.narrow(0, start_idx, shard_size))

    def forward(self, x: torch.Tensor, last_indices: Optional[torch.Tensor] = None):
        if last_indices is not None:
            x = x[last_indices].contiguous()
        logits = gemm_linear(x, self.weight, None, out_dtype=self.logits_dtype, backend=self.gemm_backend)
        if self.tp_size > 1:
            all_logits = [torch.empty_like(logits) for _ in range(self.tp_size)] if self.tp_rank == 0 else None
            dist.gather(logits, all_logits, 0)
            logits = torch.cat(all_logits, -1) if self.tp_rank == 0 else None
        return logits

    def greedy(self, x: torch.Tensor, last_indices: Optional[torch.Tensor] = None):
        """Greedy tokens without the logits: the temperature-0 branch of
        Sampler (nanovllm/layers/sampler.py:8-21, argmax of the logits read
        as fp32, first index on ties) applied to this head's output (model
        dtype, or fp32 with logits_dtype = torch.float32).  Returns (token
        ids int64, their logits as fp32); on the HIP path one fused launch
        replaces the [M, vocab] logits write and the argmax read-back.  With
        tensor parallelism every rank finds the best token of its vocabulary
        shard and rank 0 keeps the best pair, the lower rank on equal logits
        (the first index of the gathered logits); other ranks return None."""
        if last_indices is not None:
            x = x[last_indices].contiguous()
        tokens, values = greedy_linear(x, self.weight, backend=self.gemm_backend, logits_dtype=self.logits_dtype)
        if self.tp_size > 1:
            tokens = tokens + self.vocab_start_idx
            rank0 = self.tp_rank == 0
            all_tokens = [torch.empty_like(tokens) for _ in range(self.tp_size)] if rank0 else None
            all_values = [torch.empty_like(values) for _ in range(self.tp_size)] if rank0 else None
            dist.gather(tokens, all_tokens, 0)
            dist.gather(values, all_values, 0)
            if not rank0:
                return None, None
            stacked_values = torch.stack(all_values, 0)
            best = stacked_values.argmax(0, keepdim=True)
            tokens = torch.stack(all_tokens, 0).gather(0, best).squeeze(0)
            values = stacked_values.gather(0, best).squeeze(0)
        return tokens, values

    def sample(self, x: torch.Tensor, temperatures: torch.Tensor, seed: int, offset: int,
               last_indices: Optional[torch.Tensor] = None):
        """Sampler.forward (nanovllm/layers/sampler.py:8-21) on this head's
        logits: greedy tokens where temperature <= 1e-10, draws from
        softmax(logits / T) elsewhere.  On the HIP path the sampled head ranks
        each column by l / T - ln E (Gumbel-max, Philox noise at (seed,
        offset)) inside the GEMM, so no logits are written; the caller
        advances `offset` per step.  Returns token ids (and, on the HIP path,
        the winning scores; None on the torch path, which runs the
        reference Sampler on the gathered logits).  With tensor parallelism
        every rank draws for its vocabulary shard with its own key (the seed
        mixed with the rank, so shards draw independent noise), and rank 0
        keeps the best score, the lower rank on ties; other ranks return
        (None, None)."""
        if last_indices is not None:
            x = x[last_indices].contiguous()
        if self.tp_size == 1:
            return sample_linear(x, self.weight, temperatures, seed, offset, backend=self.gemm_backend,
                                 logits_dtype=self.logits_dtype)
        backend = validate_gemm_backend(self.gemm_backend) if self.gemm_backend is not None else default_backend()
        if backend == "torch" or sample_contract_reason(x, self.weight, temperatures) is not None:
            if backend == "hip":
                raise RuntimeError("HIP GEMM backend is unavailable: "
                                   f"{sample_contract_reason(x, self.weight, temperatures)}")
            logits = self.forward(x)
            return (torch_sampler(logits, temperatures), None) if self.tp_rank == 0 else (None, None)
        rank_seed = (int(seed) ^ (self.tp_rank * 0x9E3779B97F4A7C15)) & ((1 << 64) - 1)
        tokens, scores = gemm_sample(x, self.weight, temperatures, rank_seed, offset, self.logits_dtype)
        tokens = tokens + self.vocab_start_idx
        rank0 = self.tp_rank == 0
        all_tokens = [torch.empty_like(tokens) for _ in range(self.tp_size)] if rank0 else None
        all_scores = [torch.empty_like(scores) for _ in range(self.tp_size)] if rank0 else None
        dist.gather(tokens, all_tokens, 0)
        dist.gather(scores, all_scores, 0)
        if not rank0:
            return None, None
        stacked = torch.stack(all_scores, 0)
        best = stacked.argmax(0, keepdim=True)
        return torch.stack(all_tokens, 0).gather(0, best).squeeze(0), stacked.gather(0, best).squeeze(0)


class GemmLinear(nn.Linear):
    """``nn.Linear`` whose matmul goes through the backend switch; drop-in for
    the plain nn.Linear projections of nanovllm/layers/gated_delta_net.py:60-63,
    90 and nanovllm/models/qwen3_5_mtp.py:41."""

    gemm_backend: Optional[str] = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return gemm_linear(x, self.weight, self.bias, backend=self.gemm_backend)
