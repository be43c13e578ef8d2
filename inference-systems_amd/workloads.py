"""GEMM workloads of the Qwen3.5 / Qwen3 linear layers this path serves.

Shapes come from the reference's model code and GEMM bench
(paths relative to the reference repo):
  * QWEN35_SHAPES — the shape table kDefaultShapes of
    cuda_kernels/gemm/src/gemm_bench.cu:45-57 (Qwen3.5-0.8B projections,
    H = 1024: QKV N = 6144, gate_up N = 7168, out K = 2048, down K = 3584);
  * WORKLOADS — the measured problems: a square FP32 GEMM, the BF16 prefill
    projection, the BF16 decode projection for M <= 32, the FP16 long-K MLP
    down projection and the BF16 tied LM head (vocab 151936, fp32 logits,
    nanovllm/layers/embed_head.py:56-66).

Inputs are synthetic: drawn from a seeded torch CPU generator in fp32 and
rounded once (round to nearest even) to the input dtype.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

# (label, M, N, K) — gemm_bench.cu:45-57
QWEN35_SHAPES = [
    ("qwen35_decode_qkv", 1, 6144, 1024),
    ("qwen35_prefill16_qkv", 16, 6144, 1024),
    ("qwen35_prefill64_qkv", 64, 6144, 1024),
    ("qwen35_prefill256_qkv", 256, 6144, 1024),
    ("qwen35_prefill16_out", 16, 1024, 2048),
    ("qwen35_prefill64_out", 64, 1024, 2048),
    ("qwen35_prefill16_gate_up", 16, 7168, 1024),
    ("qwen35_prefill64_gate_up", 64, 7168, 1024),
    ("qwen35_prefill64_down", 64, 1024, 3584),
    ("square256", 256, 256, 256),
    ("square512", 512, 512, 512),
]


@dataclass(frozen=True)
class Workload:
    name: str
    dtype_in: torch.dtype
    dtype_out: torch.dtype
    b_layout: int            # _lib.B_NK (W[N,K]) or _lib.B_KN (B[K,N])
    ms: tuple                # M values (one problem per M)
    n: int
    k: int
    a_dist: tuple            # ("uniform", lo, hi) or ("normal", std)
    b_dist: tuple
    seed: int
    bound: str               # "mfma" (compute) or "hbm" (bandwidth)
    description: str


WORKLOADS = {
    "fp32_square_1024": Workload(
        "fp32_square_1024", torch.float32, torch.float32, _lib.B_KN, (1024,), 1024, 1024,
        ("uniform", -1.0, 1.0), ("uniform", -1.0, 1.0), 1001, "mfma",
        "FP32 C = A * B, row-major B[K,N], M = N = K = 1024"),
    "bf16_prefill_2048x4096x1024": Workload(
        "bf16_prefill_2048x4096x1024", torch.bfloat16, torch.bfloat16, _lib.B_NK, (2048,), 4096, 1024,
        ("normal", 1.0), ("normal", 0.02), 1002, "mfma",
        "BF16 prefill projection C = A * W^T, A[2048,1024], W[4096,1024], bf16 out"),
    "bf16_decode_n6144_k1024": Workload(
        "bf16_decode_n6144_k1024", torch.bfloat16, torch.bfloat16, _lib.B_NK, (1, 4, 8, 16, 32), 6144, 1024,
        ("normal", 1.0), ("normal", 0.02), 1003, "hbm",
        "BF16 decode fused projection, M in {1,4,8,16,32}, W[6144,1024], bf16 out"),
    "fp16_down_4096x1024x3584": Workload(
        "fp16_down_4096x1024x3584", torch.float16, torch.float16, _lib.B_NK, (4096,), 1024, 3584,
        ("normal", 0.5), ("normal", 0.02), 1004, "mfma",
        "FP16 MLP down projection, A[4096,3584], W[1024,3584], fp16 out"),
    "bf16_lm_head_n151936_k1024": Workload(
        "bf16_lm_head_n151936_k1024", torch.bfloat16, torch.float32, _lib.B_NK, (1, 32, 512), 151936, 1024,
        ("normal", 1.0), ("normal", 0.02), 1005, "hbm",
        "BF16 tied LM head, M in {1,32,512}, W[151936,1024], fp32 logits"),
}

HEADLINE = "bf16_prefill_2048x4096x1024"


def _draw(shape, dist, gen: torch.Generator) -> torch.Tensor:
    if dist[0] == "uniform":
        lo, hi = dist[1], dist[2]
        return torch.rand(shape, generator=gen, dtype=torch.float32) * (hi - lo) + lo
    if dist[0] == "normal":
        return torch.randn(shape, generator=gen, dtype=torch.float32) * dist[1]
    raise ValueError(dist)


def make_inputs(name: str, m: Optional[int] = None, *, seed: Optional[int] = None, n: Optional[int] = None,
                k: Optional[int] = None, device="cpu"):
    """(a, b) for a workload: a[M,K]; b is W[N,K] or B[K,N] by its layout.

    The seed is the workload's seed plus M, so each M of a multi-M workload
    has its own inputs.  `n` / `k` override the sizes (for reduced parity
    cases of the same distribution)."""
    w = WORKLOADS[name]
    m = w.ms[-1] if m is None else m
    n = w.n if n is None else n
    k = w.k if k is None else k
    gen = torch.Generator().manual_seed((w.seed if seed is None else seed) + m)
    a = _draw((m, k), w.a_dist, gen).to(w.dtype_in)
    b_shape = (n, k) if w.b_layout == _lib.B_NK else (k, n)
    b = _draw(b_shape, w.b_dist, gen).to(w.dtype_in)
    return a.to(device), b.to(device)


def problem_flops(m: int, n: int, k: int) -> float:
    """2 M N K (gemm_bench.cu:371)."""
    return 2.0 * m * n * k


def problem_bytes(m: int, n: int, k: int, dtype_in: torch.dtype, dtype_out: torch.dtype) -> float:
    """Compulsory HBM traffic: each operand read once, C written once."""
    si = torch.finfo(dtype_in).bits // 8
    so = torch.finfo(dtype_out).bits // 8
    return float((m * k + n * k) * si + m * n * so)
