"""GEMMs with a prologue on A, as PyTorch custom ops.

    gemm_gated(a[M, K], gate, w[N, K], out_dtype=None) -> out[M, N]
        out = (a * sigmoid(gate)) @ w.T, the output gate of Qwen3.5 gated
        attention followed by o_proj (nanovllm/models/qwen3_5.py:95-96).
        ``gate`` is [M, K], or the head-strided view [M, heads, head_dim]
        that ``q_proj(x).view(-1, heads, 2 * head_dim).chunk(2, -1)[1]``
        produces (qwen3_5.py:81-86); its last stride must be 1.  ``a`` may
        be the attention output [M, heads, head_dim].

    gemm_add_rmsnorm(h[M, K], residual[M, K], norm_weight[K], w, eps,
                     silu_mul=False, out_dtype=None) -> (out, residual_out)
        ``Qwen3_5RMSNorm(h, residual)`` (nanovllm/layers/layernorm.py:131-142)
        followed by the projection ``w[N, K]``, or with ``silu_mul`` by
        gate_up_proj ``w[2N, K]`` and SiluAndMul (qwen3_5.py:157-159,
        200-203, 117).  residual_out = round(h + residual) as there; the
        per-row scale rsqrt(mean s^2 + eps) is applied to the fp32 sums.
        bfloat16 inputs only (the unscaled operand s * (1 + w) needs bf16's
        exponent range).

    sigmoid_gate(a, gate) -> round(a * round(sigmoid(gate))), the gate alone.

Same conventions as ``nanovllm::gemm``: ``nanovllm`` namespace, fixed
RuntimeError messages, fake implementations, launch on the current stream,
no fallback inside the op.  ``gated_linear`` and ``add_rmsnorm_linear``
add the ``torch | hip | auto`` switch with the reference composition as the
``torch`` backend.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .. import _lib
from .gemm import _CODE, default_backend, validate_gemm_backend

_HALF = (torch.float16, torch.bfloat16)


def _flat_rows(x: torch.Tensor) -> torch.Tensor:
    """[M, ...] contiguous -> [M, prod(...)] view."""
    return x.reshape(x.shape[0], -1) if x.dim() > 2 else x


def _gate_geometry(a: torch.Tensor, gate: torch.Tensor):
    """(group, group_stride, ldg) of the gate view, or a reason string."""
    m, k = a.shape[0], a[0].numel() if a.dim() > 1 else 0
    if gate.dim() == 2:
        if tuple(gate.shape) != (m, k):
            return f"gate shape {tuple(gate.shape)} must be (M, K) = ({m}, {k})"
        if gate.stride(1) != 1:
            return "gate must have unit stride in its last dimension"
        return k, k, gate.stride(0)
    if gate.dim() == 3:
        if gate.shape[0] != m or gate.shape[1] * gate.shape[2] != k:
            return f"gate shape {tuple(gate.shape)} must be (M, heads, head_dim) with heads * head_dim = K ({k})"
        if gate.stride(2) != 1:
            return "gate must have unit stride in its last dimension"
        return gate.shape[2], gate.stride(1), gate.stride(0)
    return "gate must be (M, K) or (M, heads, head_dim)"


def gated_contract_reason(a: torch.Tensor, gate: torch.Tensor, w: torch.Tensor,
                          out_dtype: Optional[torch.dtype] = None) -> Optional[str]:
    """Why the gated GEMM cannot take these inputs, or None if it can."""
    if not (a.is_cuda and gate.is_cuda and w.is_cuda):
        return "a, gate and w must be CUDA (HIP) tensors"
    if not (a.device == gate.device == w.device):
        return "a, gate and w must be on the same device"
    if a.dtype not in _HALF:
        return "the gated GEMM takes float16 or bfloat16 inputs"
    if gate.dtype != a.dtype or w.dtype != a.dtype:
        return "a, gate and w must have the same dtype"
    if out_dtype not in (None, a.dtype, torch.float32):
        return f"out_dtype {out_dtype} is not supported for {a.dtype} inputs"
    if a.dim() < 2 or not a.is_contiguous():
        return "a must be a contiguous (M, K) or (M, heads, head_dim) tensor"
    if w.dim() != 2 or not w.is_contiguous():
        return "w must be a contiguous 2-D tensor"
    k = a[0].numel()
    if w.shape[1] != k:
        return f"w.size(1) ({w.shape[1]}) must equal K ({k})"
    geo = _gate_geometry(a, gate)
    if isinstance(geo, str):
        return geo
    group, group_stride, ldg = geo
    if k == 0 or k % 8 or group % 8 or group_stride % 8 or ldg % 8:
        return "K, head_dim and the gate strides must be multiples of 8"
    if a.data_ptr() % 16 or gate.data_ptr() % 16 or w.data_ptr() % 16:
        return "a, gate and w must be 16-byte aligned"
    return None


def _launch_gated(a, gate, w, out_dtype, kernel=None):
    reason = gated_contract_reason(a, gate, w, out_dtype)
    if reason is not None:
        raise RuntimeError(f"nanovllm::gemm_gated: {reason}")
    out_dtype = a.dtype if out_dtype is None else out_dtype
    group, group_stride, ldg = _gate_geometry(a, gate)
    m, k, n = a.shape[0], a[0].numel(), w.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=a.device)
    if m == 0 or n == 0:
        return out
    need = _lib.gated_workspace_bytes(m, k, group, _CODE[a.dtype])
    _lib.check(need if need < 0 else _lib.OK, "nanovllm_gemm_gated_workspace_bytes")
    workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=a.device)
    with torch.cuda.device(a.device):
        stream = torch.cuda.current_stream(a.device).cuda_stream
        _lib.gated_raw(a.data_ptr(), gate.data_ptr(), w.data_ptr(), out.data_ptr(), m, n, k, k, ldg, group,
                       group_stride, k, n, _CODE[a.dtype], _CODE[out_dtype], workspace.data_ptr(), need, stream,
                       kernel)
    return out


@torch.library.custom_op("nanovllm::gemm_gated", mutates_args=())
def _gemm_gated_op(a: torch.Tensor, gate: torch.Tensor, w: torch.Tensor,
                   out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    return _launch_gated(a, gate, w, out_dtype)


@_gemm_gated_op.register_fake
def _gemm_gated_fake(a, gate, w, out_dtype=None):
    torch._check(w.dim() == 2)
    torch._check(a.dim() >= 2)
    return a.new_empty((a.shape[0], w.shape[0]), dtype=a.dtype if out_dtype is None else out_dtype)


def gemm_gated(a: torch.Tensor, gate: torch.Tensor, w: torch.Tensor,
               out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """(a * sigmoid(gate)) @ w.T with the gate applied in front of the GEMM."""
    return torch.ops.nanovllm.gemm_gated(a, gate, w, out_dtype)


def gemm_gated_with_kernel(a, gate, w, kernel: int, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """The gated GEMM on a named kernel: splitk_decode fuses the gate, any
    other kernel runs after the gate kernel."""
    return _launch_gated(a, gate, w, out_dtype, kernel)


def _launch_sigmoid_gate(a, gate):
    reason = gated_contract_reason(a, gate, a.new_empty((1, a[0].numel())))
    if reason is not None:
        raise RuntimeError(f"nanovllm::sigmoid_gate: {reason}")
    group, group_stride, ldg = _gate_geometry(a, gate)
    m, k = a.shape[0], a[0].numel()
    out = torch.empty((m, k), dtype=a.dtype, device=a.device)
    if m:
        with torch.cuda.device(a.device):
            _lib.sigmoid_gate_raw(a.data_ptr(), gate.data_ptr(), out.data_ptr(), m, k, k, ldg, group, group_stride,
                                  k, _CODE[a.dtype], torch.cuda.current_stream(a.device).cuda_stream)
    return out


@torch.library.custom_op("nanovllm::sigmoid_gate", mutates_args=())
def _sigmoid_gate_op(a: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    return _launch_sigmoid_gate(a, gate)


@_sigmoid_gate_op.register_fake
def _sigmoid_gate_fake(a, gate):
    return a.new_empty((a.shape[0], a[0].numel()))


def sigmoid_gate(a: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """round(a * round(sigmoid(gate))) as [M, K]: the operand gemm_gated feeds its GEMM."""
    return torch.ops.nanovllm.sigmoid_gate(a, gate)


def add_rmsnorm_contract_reason(h: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor,
                                w: torch.Tensor, silu_mul: bool = False,
                                out_dtype: Optional[torch.dtype] = None) -> Optional[str]:
    """Why the add + RMSNorm GEMM cannot take these inputs, or None if it can."""
    tensors = (h, residual, norm_weight, w)
    if not all(t.is_cuda for t in tensors):
        return "h, residual, norm_weight and w must be CUDA (HIP) tensors"
    if len({t.device for t in tensors}) != 1:
        return "h, residual, norm_weight and w must be on the same device"
    if h.dtype != torch.bfloat16:
        # The fused norm rounds s * (1 + w) before the row scale; bf16 holds
        # that for any fp32 s, fp16 overflows or underflows where the
        # reference's normalised operand does not.
        return "the add + RMSNorm GEMM takes bfloat16 inputs"
    if any(t.dtype != h.dtype for t in tensors):
        return "h, residual, norm_weight and w must have the same dtype"
    if out_dtype not in (None, h.dtype, torch.float32):
        return f"out_dtype {out_dtype} is not supported for {h.dtype} inputs"
    if h.dim() != 2 or tuple(residual.shape) != tuple(h.shape):
        return "h and residual must be (M, K) tensors of the same shape"
    k = h.shape[1]
    if norm_weight.dim() != 1 or norm_weight.shape[0] != k:
        return f"norm_weight must be a (K,) tensor (K = {k})"
    if w.dim() != 2 or w.shape[1] != k:
        return f"w must be (N, K) with K = {k}"
    if silu_mul and (w.shape[0] % 2 or w.shape[0] == 0):
        return "with silu_mul, w must have an even, positive number of rows ([W_gate; W_up])"
    if w.shape[0] == 0:
        return "w must have at least one row"
    if not all(t.is_contiguous() for t in tensors):
        return "h, residual, norm_weight and w must be contiguous"
    if k == 0 or k % 8:
        return "K must be a positive multiple of 8"
    if any(t.data_ptr() % 16 for t in tensors):
        return "h, residual, norm_weight and w must be 16-byte aligned"
    return None


def _launch_add_rmsnorm(h, residual, norm_weight, w, eps, silu_mul, out_dtype, kernel=None):
    reason = add_rmsnorm_contract_reason(h, residual, norm_weight, w, silu_mul, out_dtype)
    if reason is not None:
        raise RuntimeError(f"nanovllm::gemm_add_rmsnorm: {reason}")
    out_dtype = h.dtype if out_dtype is None else out_dtype
    m, k = h.shape
    n = w.shape[0] // 2 if silu_mul else w.shape[0]
    out = torch.empty((m, n), dtype=out_dtype, device=h.device)
    residual_out = torch.empty_like(h)
    if m == 0:
        return out, residual_out
    need = _lib.add_rmsnorm_workspace_bytes(m, k, _CODE[h.dtype])
    _lib.check(need if need < 0 else _lib.OK, "nanovllm_gemm_add_rmsnorm_workspace_bytes")
    workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=h.device)
    with torch.cuda.device(h.device):
        stream = torch.cuda.current_stream(h.device).cuda_stream
        _lib.add_rmsnorm_raw(h.data_ptr(), residual.data_ptr(), norm_weight.data_ptr(), float(eps), w.data_ptr(),
                             out.data_ptr(), residual_out.data_ptr(), m, n, k, k, k, k, n, k, silu_mul,
                             _CODE[h.dtype], _CODE[out_dtype], workspace.data_ptr(), need, stream, kernel)
    return out, residual_out


@torch.library.custom_op("nanovllm::gemm_add_rmsnorm", mutates_args=())
def _gemm_add_rmsnorm_op(h: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor, w: torch.Tensor,
                         eps: float, silu_mul: bool = False,
                         out_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    return _launch_add_rmsnorm(h, residual, norm_weight, w, eps, silu_mul, out_dtype)


@_gemm_add_rmsnorm_op.register_fake
def _gemm_add_rmsnorm_fake(h, residual, norm_weight, w, eps, silu_mul=False, out_dtype=None):
    torch._check(h.dim() == 2 and w.dim() == 2)
    n = w.shape[0] // 2 if silu_mul else w.shape[0]
    return (h.new_empty((h.shape[0], n), dtype=h.dtype if out_dtype is None else out_dtype), torch.empty_like(h))


def gemm_add_rmsnorm(h: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor, w: torch.Tensor,
                     eps: float, silu_mul: bool = False,
                     out_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(projection of RMSNorm(h + residual), round(h + residual))."""
    return torch.ops.nanovllm.gemm_add_rmsnorm(h, residual, norm_weight, w, float(eps), bool(silu_mul), out_dtype)


def gemm_add_rmsnorm_with_kernel(h, residual, norm_weight, w, eps, kernel: int, silu_mul: bool = False,
                                 out_dtype: Optional[torch.dtype] = None):
    """The add + RMSNorm GEMM on splitk_decode (fused) or mfma_staged
    (prologue kernel, then row-scaled GEMM)."""
    return _launch_add_rmsnorm(h, residual, norm_weight, w, eps, silu_mul, out_dtype, kernel)


# ---------------------------------------------------------------------------
# Backend switch and the reference compositions
# ---------------------------------------------------------------------------
def _torch_gated(x, gate, weight):
    """`output * torch.sigmoid(gate)` then o_proj (qwen3_5.py:95-96)."""
    m = x.shape[0]
    g = gate.reshape(m, -1) if gate.dim() == 2 else gate
    gated = (x.reshape(g.shape) * torch.sigmoid(g)).reshape(m, -1)
    return F.linear(gated, weight)


def gated_linear(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, *,
                 backend: Optional[str] = None) -> torch.Tensor:
    """F.linear(x * sigmoid(gate), weight) with the backend switch of ``linear``."""
    backend = validate_gemm_backend(backend) if backend is not None else default_backend()
    if backend != "torch":
        reason = gated_contract_reason(x, gate, weight)
        if reason is None:
            return gemm_gated(x, gate, weight)
        if backend == "hip":
            raise RuntimeError(f"HIP GEMM backend is unavailable: {reason}")
    return _torch_gated(x, gate, weight)


def torch_add_rmsnorm(h: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor, eps: float):
    """Qwen3_5RMSNorm.forward(h, residual) (nanovllm/layers/layernorm.py:131-142)."""
    summed = h.float() + residual.float()
    new_residual = summed.to(h.dtype)
    variance = summed.pow(2).mean(dim=-1, keepdim=True)
    normalized = summed * torch.rsqrt(variance + eps) * (1.0 + norm_weight.float())
    return normalized.to(h.dtype), new_residual


def add_rmsnorm_linear(h: torch.Tensor, residual: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                       weight: torch.Tensor, *, silu_mul: bool = False,
                       backend: Optional[str] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(F.linear(norm(h + residual), weight) [then SiluAndMul], new residual)
    with the backend switch of ``linear``."""
    backend = validate_gemm_backend(backend) if backend is not None else default_backend()
    if backend != "torch":
        reason = add_rmsnorm_contract_reason(h, residual, norm_weight, weight, silu_mul)
        if reason is None:
            return gemm_add_rmsnorm(h, residual, norm_weight, weight, eps, silu_mul)
        if backend == "hip":
            raise RuntimeError(f"HIP GEMM backend is unavailable: {reason}")
    normed, new_residual = torch_add_rmsnorm(h, residual, norm_weight, eps)
    y = F.linear(normed, weight)
    if silu_mul:
        gate, up = y.chunk(2, -1)
        y = F.silu(gate) * up
    return y, new_residual
