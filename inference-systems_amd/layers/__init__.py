"""nano-vLLM layer mirrors whose matmul is the MI355X GEMM (see linear.py and
gdn_projection.py)."""
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

__all__ = [
    "ColumnParallelLinear",
    "GdnInputProjection",
    "GemmLinear",
    "LinearBase",
    "MergedColumnParallelLinear",
    "ParallelLMHead",
    "QKVParallelLinear",
    "ReplicatedLinear",
    "RowParallelLinear",
]
