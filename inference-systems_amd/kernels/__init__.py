"""Op wrappers (layout of nanovllm/kernels/__init__.py): the GEMM custom op."""
from .gemm import (
    contract_reason,
    gemm,
    gemm_kn,
    gemm_with_kernel,
    linear,
    selected_kernel,
    validate_gemm_backend,
)

__all__ = [
    "contract_reason",
    "gemm",
    "gemm_kn",
    "gemm_with_kernel",
    "linear",
    "selected_kernel",
    "validate_gemm_backend",
]
