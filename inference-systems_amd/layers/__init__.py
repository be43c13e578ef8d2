"""nano-vLLM layer mirrors whose matmul is the MI355X GEMM (see linear.py,
gdn_projection.py and mlp.py)."""
from .gdn_projection import GdnInputProjection
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
from .mlp import Qwen35MLP

__all__ = [
    "ColumnParallelLinear",
    "GdnInputProjection",
    "GemmLinear",
    "LinearBase",
    "MergedColumnParallelLinear",
    "ParallelLMHead",
    "QKVParallelLinear",
    "Qwen35MLP",
    "ReplicatedLinear",
    "RowParallelLinear",
]
