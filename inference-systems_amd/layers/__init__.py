"""nano-vLLM layer mirrors whose matmul is the MI355X GEMM (see linear.py)."""
from .linear import (
    ColumnParallelLinear,
    GemmLinear,
    LinearBase,
    MergedColumnParallelLinear,
    ParallelLMHead,
    QKVParallelLinear,
    ReplicatedLinear,
    RowParallelLinear,
)

__all__ = [
    "ColumnParallelLinear",
    "GemmLinear",
    "LinearBase",
    "MergedColumnParallelLinear",
    "ParallelLMHead",
    "QKVParallelLinear",
    "ReplicatedLinear",
    "RowParallelLinear",
]
