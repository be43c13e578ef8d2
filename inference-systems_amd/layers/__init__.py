"""nano-vLLM layer mirrors whose matmul is the MI355X GEMM (see linear.py,
gdn_projection.py and mlp.py) and the Qwen3.5 RMSNorm (norm.py)."""
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
from .norm import Qwen35RMSNorm

__all__ = [
    "ColumnParallelLinear",
    "GdnInputProjection",
    "GemmLinear",
    "LinearBase",
    "MergedColumnParallelLinear",
    "ParallelLMHead",
    "QKVParallelLinear",
    "Qwen35MLP",
    "Qwen35RMSNorm",
    "ReplicatedLinear",
    "RowParallelLinear",
]
