"""Op wrappers (layout of nanovllm/kernels/__init__.py): the GEMM custom ops."""
from .gemm import (
    contract_reason,
    gemm,
    gemm_kn,
    gemm_silu_mul,
    gemm_silu_mul_with_kernel,
    gemm_with_kernel,
    linear,
    selected_kernel,
    silu_mul_contract_reason,
    silu_mul_linear,
    silu_mul_selected_kernel,
    validate_gemm_backend,
)

__all__ = [
    "contract_reason",
    "gemm",
    "gemm_kn",
    "gemm_silu_mul",
    "gemm_silu_mul_with_kernel",
    "gemm_with_kernel",
    "linear",
    "selected_kernel",
    "silu_mul_contract_reason",
    "silu_mul_linear",
    "silu_mul_selected_kernel",
    "validate_gemm_backend",
]
