"""``nanovllm::gemm`` — the shape-aware MI355X GEMM as a PyTorch custom op.

Contract (the F.linear contract of nanovllm/layers/linear.py:51,73,153 and
nanovllm/layers/embed_head.py:61, without the bias):

    gemm(a[..., K], w[N, K], out_dtype=None) -> out[..., N]
    out = a @ w.T, accumulated in fp32, stored as out_dtype (default a.dtype)

Supported (in -> out): fp32 -> fp32, fp16 -> {fp16, fp32},
bf16 -> {bf16, fp32}.  ``gemm_kn(a[..., K], b[K, N])`` is the same op for a
row-major B[K, N] (the layout of cuda_kernels/gemm/src/gemm_bench.cu:103-106
and gemm_tiled.cu:16).

The op follows the reference's custom-op conventions:
  * schema in the ``nanovllm`` namespace (nanovllm/csrc/ops.cpp:48-71);
  * argument checks that raise ``RuntimeError`` with a fixed message, like
    the TORCH_CHECKs of nanovllm/csrc/add_kernel.cu:49-63 ("... must be
    contiguous", "... same dtype", ...);
  * a fake (meta) implementation for torch.compile (nanovllm/kernels/add.py:11-16);
  * launch on PyTorch's current stream of the input's device
    (add_kernel.cu:65-67), so the op is graph-capturable;
  * a ``torch | hip | auto`` backend switch with a contract-reason check
    (nanovllm/kernels/gdn.py:138-259), in ``linear`` below.

The HIP path has no substitute: if the native library is missing the op
raises, and ``auto`` only routes to ``F.linear`` for inputs outside the
op's contract (CPU tensors, unsupported dtypes), never because the library
could not be loaded.
"""
from __future__ import annotations

import os
from pathlib import Path
from typing import Optional

import torch
import torch.nn.functional as F

from .. import _lib

_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}
_OUT_OK = {
    torch.float32: (torch.float32,),
    torch.float16: (torch.float16, torch.float32),
    torch.bfloat16: (torch.bfloat16, torch.float32),
}

BACKENDS = ("torch", "hip", "auto")
BACKEND_ENV = "NANOVLLM_GEMM_BACKEND"


def contract_reason(a: torch.Tensor, b: torch.Tensor, out_dtype: Optional[torch.dtype] = None,
                    b_layout: int = _lib.B_NK) -> Optional[str]:
    """Why the HIP op cannot take these inputs, or None if it can."""
    if not (a.is_cuda and b.is_cuda):
        return "a and w must be CUDA (HIP) tensors"
    if a.device != b.device:
        return "a and w must be on the same device"
    if a.dtype not in _CODE:
        return "a must be float32, float16 or bfloat16"
    if b.dtype != a.dtype:
        return "a and w must have the same dtype"
    out = a.dtype if out_dtype is None else out_dtype
    if out not in _OUT_OK[a.dtype]:
        return f"out_dtype {out} is not supported for {a.dtype} inputs"
    if b.dim() != 2:
        return "w must be 2-D"
    if a.dim() < 1:
        return "a must have at least one dimension"
    k = b.shape[1] if b_layout == _lib.B_NK else b.shape[0]
    if a.shape[-1] != k:
        what = "w.size(1)" if b_layout == _lib.B_NK else "b.size(0)"
        return f"a.size(-1) ({a.shape[-1]}) must equal {what} ({k})"
    if k == 0:
        return "K must be positive"
    if not a.is_contiguous():
        return "a must be contiguous"
    if not b.is_contiguous():
        return "w must be contiguous"
    return None


def _launch(a: torch.Tensor, b: torch.Tensor, out_dtype: Optional[torch.dtype], b_layout: int,
            kernel: Optional[int] = None) -> torch.Tensor:
    reason = contract_reason(a, b, out_dtype, b_layout)
    if reason is not None:
        raise RuntimeError(f"nanovllm::gemm: {reason}")
    out_dtype = a.dtype if out_dtype is None else out_dtype
    k = a.shape[-1]
    n = b.shape[0] if b_layout == _lib.B_NK else b.shape[1]
    m = a.numel() // k
    out = torch.empty((*a.shape[:-1], n), dtype=out_dtype, device=a.device)
    if m == 0 or n == 0:
        return out
    with torch.cuda.device(a.device):
        stream = torch.cuda.current_stream(a.device).cuda_stream
        ldb = k if b_layout == _lib.B_NK else n
        _lib.gemm_raw(a.data_ptr(), b.data_ptr(), out.data_ptr(), m, n, k, k, ldb, n, b_layout,
                      _CODE[a.dtype], _CODE[out_dtype], stream, kernel)
    return out


# ---------------------------------------------------------------------------
# Registration of nanovllm::gemm / nanovllm::gemm_kn
# ---------------------------------------------------------------------------
# Two registrations of the same schemas over the same C ABI:
#   torch_library  csrc/torch_ops.cpp, a TORCH_LIBRARY fragment built into
#                  libnanovllm_torch_ops.so (the nanovllm/csrc/ops.cpp:48-80
#                  pattern); the dispatcher calls C++ directly.
#   custom_op      torch.library.custom_op over the ctypes binding below.
# The default is torch_library when that library is built (it costs less
# host time per eager call) and custom_op otherwise; NANOVLLM_GEMM_OPS
# picks one.  Both raise the same messages; neither has a CPU fallback.
OPS_ENV = "NANOVLLM_GEMM_OPS"
REGISTRATIONS = ("torch_library", "custom_op")
TORCH_OPS_LIB = Path(_lib.__file__).resolve().parent / "libnanovllm_torch_ops.so"


def _choose_registration() -> str:
    asked = os.environ.get(OPS_ENV, "").strip().lower()
    if asked and asked not in REGISTRATIONS:
        raise ValueError(f"{OPS_ENV} must be one of {REGISTRATIONS}, got {asked!r}")
    # The C++ registration links the in-tree libnanovllm_gemm.so; a library
    # named by NANOVLLM_GEMM_LIB (a sanitized build) goes through ctypes.
    usable = TORCH_OPS_LIB.is_file() and _lib.LIB_PATH.is_file() and _lib.library_path() == _lib.LIB_PATH
    if asked == "torch_library":
        if not usable:
            raise _lib.GemmLibraryError(
                f"{OPS_ENV}=torch_library needs {TORCH_OPS_LIB.name} and {_lib.LIB_PATH.name} built in "
                f"{TORCH_OPS_LIB.parent} (and NANOVLLM_GEMM_LIB unset)")
        return asked
    if asked == "custom_op":
        return asked
    return "torch_library" if usable else "custom_op"


REGISTRATION = _choose_registration()
if REGISTRATION == "torch_library":
    try:
        torch.ops.load_library(str(TORCH_OPS_LIB))
    except (OSError, RuntimeError) as exc:
        # Asked for by name: fail.  By default: the custom_op registration
        # below reaches the same kernels through ctypes.
        if os.environ.get(OPS_ENV, "").strip().lower() == "torch_library":
            raise _lib.GemmLibraryError(f"failed to load {TORCH_OPS_LIB}: {exc}") from exc
        import warnings

        warnings.warn(f"{TORCH_OPS_LIB.name} did not load ({exc}); registering nanovllm::gemm through ctypes",
                      RuntimeWarning, stacklevel=2)
        REGISTRATION = "custom_op"


def _gemm_fake(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    torch._check(w.dim() == 2)
    torch._check(a.shape[-1] == w.shape[1])
    torch._check(a.dtype == w.dtype)
    torch._check(a.device == w.device)
    return a.new_empty((*a.shape[:-1], w.shape[0]), dtype=a.dtype if out_dtype is None else out_dtype)


def _gemm_kn_fake(a: torch.Tensor, b: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    torch._check(b.dim() == 2)
    torch._check(a.shape[-1] == b.shape[0])
    torch._check(a.dtype == b.dtype)
    torch._check(a.device == b.device)
    return a.new_empty((*a.shape[:-1], b.shape[1]), dtype=a.dtype if out_dtype is None else out_dtype)


if REGISTRATION == "torch_library":
    torch.library.register_fake("nanovllm::gemm")(_gemm_fake)
    torch.library.register_fake("nanovllm::gemm_kn")(_gemm_kn_fake)
else:
    @torch.library.custom_op("nanovllm::gemm", mutates_args=())
    def _gemm_op(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        return _launch(a, w, out_dtype, _lib.B_NK)

    @torch.library.custom_op("nanovllm::gemm_kn", mutates_args=())
    def _gemm_kn_op(a: torch.Tensor, b: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        return _launch(a, b, out_dtype, _lib.B_KN)

    _gemm_op.register_fake(_gemm_fake)
    _gemm_kn_op.register_fake(_gemm_kn_fake)


def gemm(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """a @ w.T on the MI355X kernels (w in nn.Linear [N, K] layout)."""
    return torch.ops.nanovllm.gemm(a, w, out_dtype)


def gemm_kn(a: torch.Tensor, b: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """a @ b on the MI355X kernels (b row-major [K, N])."""
    return torch.ops.nanovllm.gemm_kn(a, b, out_dtype)


def gemm_with_kernel(a: torch.Tensor, b: torch.Tensor, kernel: int, out_dtype: Optional[torch.dtype] = None,
                     b_layout: int = _lib.B_NK) -> torch.Tensor:
    """Run one named kernel of the ladder (raises if it cannot take the shape)."""
    return _launch(a, b, out_dtype, b_layout, kernel)


def selected_kernel(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype] = None,
                    b_layout: int = _lib.B_NK) -> str:
    """Name of the kernel the selection table picks for these operands."""
    k = a.shape[-1]
    n = w.shape[0] if b_layout == _lib.B_NK else w.shape[1]
    m = a.numel() // max(k, 1)
    out_dtype = a.dtype if out_dtype is None else out_dtype
    aligned = a.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0
    ldb = k if b_layout == _lib.B_NK else n
    kid = _lib.select(m, n, k, k, ldb, n, b_layout, _CODE[a.dtype], _CODE[out_dtype], aligned)
    if kid < 0:
        raise RuntimeError(f"nanovllm::gemm: {_lib.last_error()}")
    return _lib.kernel_name(kid)


# ---------------------------------------------------------------------------
# Fused gate/up projection + SiLU-and-mul
# ---------------------------------------------------------------------------
def silu_mul_contract_reason(a: torch.Tensor, w: torch.Tensor,
                             out_dtype: Optional[torch.dtype] = None) -> Optional[str]:
    """Why the fused op cannot take these inputs, or None if it can: the
    GEMM contract, half-precision inputs, an even number of W rows (gate
    rows, then as many up rows) and rows readable as aligned 16-byte chunks."""
    reason = contract_reason(a, w, out_dtype)
    if reason is not None:
        return reason
    if a.dtype not in (torch.float16, torch.bfloat16):
        return "the fused SiLU-and-mul takes float16 or bfloat16 inputs"
    if w.shape[0] % 2:
        return f"w must hold gate and up halves of equal height (got {w.shape[0]} rows)"
    if a.shape[-1] % 8:
        return f"K ({a.shape[-1]}) must be a multiple of 8 for the fused SiLU-and-mul"
    if a.data_ptr() % 16 or w.data_ptr() % 16:
        return "a and w must be 16-byte aligned for the fused SiLU-and-mul"
    return None


def _launch_silu_mul(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype],
                     kernel: Optional[int] = None) -> torch.Tensor:
    reason = silu_mul_contract_reason(a, w, out_dtype)
    if reason is not None:
        raise RuntimeError(f"nanovllm::gemm_silu_mul: {reason}")
    out_dtype = a.dtype if out_dtype is None else out_dtype
    k = a.shape[-1]
    n = w.shape[0] // 2
    m = a.numel() // k
    out = torch.empty((*a.shape[:-1], n), dtype=out_dtype, device=a.device)
    if m == 0 or n == 0:
        return out
    with torch.cuda.device(a.device):
        stream = torch.cuda.current_stream(a.device).cuda_stream
        _lib.silu_mul_raw(a.data_ptr(), w.data_ptr(), out.data_ptr(), m, n, k, k, k, n, _CODE[a.dtype],
                          _CODE[out_dtype], stream, kernel)
    return out


@torch.library.custom_op("nanovllm::gemm_silu_mul", mutates_args=())
def _gemm_silu_mul_op(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    return _launch_silu_mul(a, w, out_dtype)


@_gemm_silu_mul_op.register_fake
def _gemm_silu_mul_fake(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    torch._check(w.dim() == 2)
    torch._check(w.shape[0] % 2 == 0)
    torch._check(a.shape[-1] == w.shape[1])
    torch._check(a.dtype == w.dtype)
    torch._check(a.device == w.device)
    return a.new_empty((*a.shape[:-1], w.shape[0] // 2), dtype=a.dtype if out_dtype is None else out_dtype)


def gemm_silu_mul(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """SiluAndMul(a @ w.T) in one launch: silu(a W_gate^T) * (a W_up^T) for
    w = [W_gate; W_up] (the gate_up_proj weight)."""
    return torch.ops.nanovllm.gemm_silu_mul(a, w, out_dtype)


def gemm_silu_mul_with_kernel(a: torch.Tensor, w: torch.Tensor, kernel: int,
                              out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """The fused op on one named kernel (raises if it cannot take the shape)."""
    return _launch_silu_mul(a, w, out_dtype, kernel)


def silu_mul_selected_kernel(a: torch.Tensor, w: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> str:
    k = a.shape[-1]
    n = w.shape[0] // 2
    m = a.numel() // max(k, 1)
    out_dtype = a.dtype if out_dtype is None else out_dtype
    aligned = a.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0
    kid = _lib.silu_mul_select(m, n, k, k, k, n, _CODE[a.dtype], _CODE[out_dtype], aligned)
    if kid < 0:
        raise RuntimeError(f"nanovllm::gemm_silu_mul: {_lib.last_error()}")
    return _lib.kernel_name(kid)


# ---------------------------------------------------------------------------
# Greedy LM head: argmax of a @ w.T per row without the logits
# ---------------------------------------------------------------------------
def argmax_contract_reason(a: torch.Tensor, w: torch.Tensor) -> Optional[str]:
    """Why the greedy head cannot take these inputs, or None if it can."""
    reason = contract_reason(a, w, torch.float32 if a.dtype != torch.float32 else None)
    if reason is not None:
        return reason
    if a.dtype not in (torch.float16, torch.bfloat16):
        return "the greedy head takes float16 or bfloat16 inputs"
    if w.shape[0] < 1:
        return "w must have at least one row (vocabulary entry)"
    if a.shape[-1] % 8:
        return f"K ({a.shape[-1]}) must be a multiple of 8 for the greedy head"
    if a.data_ptr() % 16 or w.data_ptr() % 16:
        return "a and w must be 16-byte aligned for the greedy head"
    return None


def _logit_code(a: torch.Tensor, logits_dtype: Optional[torch.dtype], op: str) -> int:
    """The C ABI's logit_dtype: None or a.dtype ranks the logits rounded to
    the input type (what the reference's F.linear hands to its sampler,
    nanovllm/layers/embed_head.py:61, sampler.py:15), float32 the fp32 sums."""
    if logits_dtype is None or logits_dtype == a.dtype:
        return _CODE[a.dtype]
    if logits_dtype == torch.float32:
        return _lib.F32
    raise RuntimeError(f"nanovllm::{op}: logits_dtype must be None, {a.dtype} or torch.float32, got {logits_dtype}")


def _launch_argmax(a: torch.Tensor, w: torch.Tensor, logits_dtype: Optional[torch.dtype] = None,
                   kernel: Optional[int] = None):
    reason = argmax_contract_reason(a, w)
    if reason is not None:
        raise RuntimeError(f"nanovllm::gemm_argmax: {reason}")
    code = _logit_code(a, logits_dtype, "gemm_argmax")
    k = a.shape[-1]
    n = w.shape[0]
    m = a.numel() // k
    tokens = torch.empty(a.shape[:-1], dtype=torch.int64, device=a.device)
    logits = torch.empty(a.shape[:-1], dtype=torch.float32, device=a.device)
    if m == 0:
        return tokens, logits
    need = _lib.argmax_workspace_bytes(m, n, k, k, k, _CODE[a.dtype])
    _lib.check(need if need < 0 else _lib.OK, "nanovllm_gemm_argmax_workspace_bytes")
    workspace = torch.empty(need, dtype=torch.uint8, device=a.device)
    with torch.cuda.device(a.device):
        stream = torch.cuda.current_stream(a.device).cuda_stream
        _lib.argmax_raw(a.data_ptr(), w.data_ptr(), tokens.data_ptr(), logits.data_ptr(), m, n, k, k, k,
                        _CODE[a.dtype], code, workspace.data_ptr(), need, stream, kernel)
    return tokens, logits


@torch.library.custom_op("nanovllm::gemm_argmax", mutates_args=())
def _gemm_argmax_op(a: torch.Tensor, w: torch.Tensor,
                    logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    return _launch_argmax(a, w, logits_dtype)


@_gemm_argmax_op.register_fake
def _gemm_argmax_fake(a: torch.Tensor, w: torch.Tensor,
                      logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    torch._check(w.dim() == 2)
    torch._check(a.shape[-1] == w.shape[1])
    torch._check(a.dtype == w.dtype)
    torch._check(a.device == w.device)
    return (a.new_empty(a.shape[:-1], dtype=torch.int64), a.new_empty(a.shape[:-1], dtype=torch.float32))


def gemm_argmax(a: torch.Tensor, w: torch.Tensor,
                logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(argmax_j L(a @ w.T)[..., j], that L as fp32), without the logits;
    ties go to the first index, as in torch.argmax.  L is the logit rounded
    to a.dtype (logits_dtype None or a.dtype: the reference's greedy token
    on the logits F.linear returns in the model dtype) or the fp32 sum
    itself (logits_dtype=torch.float32)."""
    return torch.ops.nanovllm.gemm_argmax(a, w, logits_dtype)


def gemm_argmax_with_kernel(a: torch.Tensor, w: torch.Tensor, kernel: int,
                            logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The greedy head with its GEMM pass on one named kernel."""
    return _launch_argmax(a, w, logits_dtype, kernel)


# ---------------------------------------------------------------------------
# Sampled LM head: Sampler.forward on a @ w.T without the logits
# ---------------------------------------------------------------------------
def sample_contract_reason(a: torch.Tensor, w: torch.Tensor, temperatures: torch.Tensor) -> Optional[str]:
    """Why the sampled head cannot take these inputs, or None if it can."""
    reason = argmax_contract_reason(a, w)
    if reason is not None:
        return reason
    if temperatures.dtype != torch.float32:
        return f"temperatures must be float32, got {temperatures.dtype}"
    if temperatures.device != a.device:
        return "temperatures must be on the device of a"
    if temperatures.shape != a.shape[:-1]:
        return f"temperatures must have shape {tuple(a.shape[:-1])}, got {tuple(temperatures.shape)}"
    if not temperatures.is_contiguous():
        return "temperatures must be contiguous"
    return None


def _launch_sample(a: torch.Tensor, w: torch.Tensor, temperatures: torch.Tensor, seed: int, offset: int,
                   logits_dtype: Optional[torch.dtype] = None, kernel: Optional[int] = None):
    reason = sample_contract_reason(a, w, temperatures)
    if reason is not None:
        raise RuntimeError(f"nanovllm::gemm_sample: {reason}")
    code = _logit_code(a, logits_dtype, "gemm_sample")
    k = a.shape[-1]
    n = w.shape[0]
    m = a.numel() // k
    tokens = torch.empty(a.shape[:-1], dtype=torch.int64, device=a.device)
    scores = torch.empty(a.shape[:-1], dtype=torch.float32, device=a.device)
    if m == 0:
        return tokens, scores
    need = _lib.argmax_workspace_bytes(m, n, k, k, k, _CODE[a.dtype])
    _lib.check(need if need < 0 else _lib.OK, "nanovllm_gemm_argmax_workspace_bytes")
    workspace = torch.empty(need, dtype=torch.uint8, device=a.device)
    with torch.cuda.device(a.device):
        stream = torch.cuda.current_stream(a.device).cuda_stream
        _lib.sample_raw(a.data_ptr(), w.data_ptr(), temperatures.data_ptr(), int(seed), int(offset),
                        tokens.data_ptr(), scores.data_ptr(), m, n, k, k, k, _CODE[a.dtype], code,
                        workspace.data_ptr(), need, stream, kernel)
    return tokens, scores


@torch.library.custom_op("nanovllm::gemm_sample", mutates_args=())
def _gemm_sample_op(a: torch.Tensor, w: torch.Tensor, temperatures: torch.Tensor, seed: int,
                    offset: int, logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    return _launch_sample(a, w, temperatures, seed, offset, logits_dtype)


@_gemm_sample_op.register_fake
def _gemm_sample_fake(a: torch.Tensor, w: torch.Tensor, temperatures: torch.Tensor, seed: int,
                      offset: int, logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    torch._check(w.dim() == 2)
    torch._check(a.shape[-1] == w.shape[1])
    torch._check(a.dtype == w.dtype)
    torch._check(a.device == w.device)
    torch._check(temperatures.shape == a.shape[:-1])
    return (a.new_empty(a.shape[:-1], dtype=torch.int64), a.new_empty(a.shape[:-1], dtype=torch.float32))


def _as_i64(x: int) -> int:
    """x modulo 2^64 as a signed 64-bit value (the op schema's int), the
    same 64 bits the C ABI reads as uint64_t."""
    x = int(x) & ((1 << 64) - 1)
    return x - (1 << 64) if x >= 1 << 63 else x


def gemm_sample(a: torch.Tensor, w: torch.Tensor, temperatures: torch.Tensor, seed: int,
                offset: int, logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Sampler.forward (nanovllm/layers/sampler.py:8-21) on the logits
    a @ w.T (rounded to a.dtype as the reference's F.linear returns them,
    or fp32 with logits_dtype=torch.float32, as gemm_argmax ranks them)
    without writing them: (token ids, winning scores).  Rows with
    temperature <= 1e-10 take the greedy token (score = its logit); the
    others a draw from softmax(logits / T) by the Gumbel-max rule
    argmax_j (l_j / T - ln E_j), the reference's argmax of
    softmax(l / T) / E, with E from the library's Philox4x32-10 stream at
    (seed, offset), both taken modulo 2^64; advance `offset` between calls
    for fresh draws."""
    return torch.ops.nanovllm.gemm_sample(a, w, temperatures, _as_i64(seed), _as_i64(offset), logits_dtype)


def gemm_sample_with_kernel(a: torch.Tensor, w: torch.Tensor, temperatures: torch.Tensor, seed: int, offset: int,
                            kernel: int, logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """The sampled head with its GEMM pass on one named kernel."""
    return _launch_sample(a, w, temperatures, seed, offset, logits_dtype, kernel)


def validate_gemm_backend(backend: str) -> str:
    """Normalise a backend name (pattern of validate_gdn_decode_backend, gdn.py:13)."""
    value = str(backend).strip().lower()
    if value not in BACKENDS:
        raise ValueError(f"GEMM backend must be one of {BACKENDS}, got {backend!r}")
    return value


def default_backend() -> str:
    return validate_gemm_backend(os.environ.get(BACKEND_ENV, "torch"))


def _torch_linear(x, weight, bias, out_dtype):
    y = F.linear(x, weight, bias)
    return y if out_dtype is None or y.dtype == out_dtype else y.to(out_dtype)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
           out_dtype: Optional[torch.dtype] = None, backend: Optional[str] = None) -> torch.Tensor:
    """Drop-in for ``F.linear(x, weight, bias)`` with a backend switch.

    ``torch``: F.linear.  ``hip``: the nanovllm::gemm op; inputs outside its
    contract raise.  ``auto``: the op when the inputs satisfy its contract,
    F.linear otherwise (e.g. CPU tensors).  The bias is added after the GEMM.
    """
    backend = validate_gemm_backend(backend) if backend is not None else default_backend()
    if backend == "torch":
        return _torch_linear(x, weight, bias, out_dtype)
    reason = contract_reason(x, weight, out_dtype)
    if reason is not None:
        if backend == "auto":
            return _torch_linear(x, weight, bias, out_dtype)
        raise RuntimeError(f"HIP GEMM backend is unavailable: {reason}")
    y = gemm(x, weight, out_dtype)
    if bias is not None:
        y = y + bias.to(y.dtype)
    return y


def _torch_silu_mul(x, weight):
    """The reference composition: gate_up_proj then SiluAndMul
    (nanovllm/models/qwen3_5.py:117, nanovllm/layers/activation.py:8-11)."""
    gate, up = F.linear(x, weight).chunk(2, -1)
    return F.silu(gate) * up


def silu_mul_linear(x: torch.Tensor, weight: torch.Tensor, *, backend: Optional[str] = None) -> torch.Tensor:
    """SiluAndMul(F.linear(x, weight)) with the backend switch of ``linear``:
    ``torch`` runs the reference composition, ``hip`` the fused op (inputs
    outside its contract raise), ``auto`` the fused op when the inputs
    satisfy its contract and the composition otherwise."""
    backend = validate_gemm_backend(backend) if backend is not None else default_backend()
    if backend == "torch":
        return _torch_silu_mul(x, weight)
    reason = silu_mul_contract_reason(x, weight)
    if reason is not None:
        if backend == "auto":
            return _torch_silu_mul(x, weight)
        raise RuntimeError(f"HIP GEMM backend is unavailable: {reason}")
    return gemm_silu_mul(x, weight)


def _torch_logits(x, weight, logits_dtype):
    """The logits the torch path ranks, as fp32: F.linear in the model dtype
    (the reference's ParallelLMHead), or an fp32 GEMM of the same inputs."""
    if logits_dtype == torch.float32 and x.dtype != torch.float32:
        return F.linear(x.float(), weight.float())
    return F.linear(x, weight).float()


def greedy_linear(x: torch.Tensor, weight: torch.Tensor, *, backend: Optional[str] = None,
                  logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(argmax, max) of the logits F.linear(x, weight) along the last dim,
    read as fp32, with the backend switch of ``linear``: ``torch`` computes
    the logits and takes torch.argmax (Sampler's greedy branch,
    sampler.py:8-21), ``hip`` runs the fused greedy head, ``auto`` the fused
    head when its contract holds.  logits_dtype None (or x.dtype) ranks the
    logits in the model dtype, as the reference does; torch.float32 ranks
    fp32 logits."""
    backend = validate_gemm_backend(backend) if backend is not None else default_backend()
    if backend != "torch":
        reason = argmax_contract_reason(x, weight)
        if reason is None:
            return gemm_argmax(x, weight, logits_dtype)
        if backend == "hip":
            raise RuntimeError(f"HIP GEMM backend is unavailable: {reason}")
    logits = _torch_logits(x, weight, logits_dtype)
    tokens = logits.argmax(dim=-1)
    return tokens, logits.gather(-1, tokens.unsqueeze(-1)).squeeze(-1)


def torch_sampler(logits: torch.Tensor, temperatures: torch.Tensor) -> torch.Tensor:
    """Sampler.forward (nanovllm/layers/sampler.py:8-21) as the reference
    writes it, with torch's exponential draws: the ``torch`` backend of
    sample_linear and the unfused baseline of the bench."""
    greedy = temperatures <= 1e-10
    safe_temperatures = torch.where(greedy, torch.ones_like(temperatures), temperatures)
    float_logits = logits.float()
    probs = torch.softmax(float_logits / safe_temperatures.unsqueeze(dim=1), dim=-1)
    sample_tokens = probs.div_(torch.empty_like(probs).exponential_(1).clamp_min_(1e-10)).argmax(dim=-1)
    return torch.where(greedy, float_logits.argmax(dim=-1), sample_tokens)


def sample_linear(x: torch.Tensor, weight: torch.Tensor, temperatures: torch.Tensor, seed: int, offset: int, *,
                  backend: Optional[str] = None,
                  logits_dtype: Optional[torch.dtype] = None) -> tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Sampled tokens of F.linear(x, weight) with the backend switch of
    ``linear``: ``torch`` writes the logits (model dtype, or fp32 with
    logits_dtype=torch.float32) and runs the reference Sampler (its own
    exponential draws; no scores, None), ``hip`` the fused sampled head,
    ``auto`` the fused head when its contract holds.  Returns (tokens,
    scores)."""
    backend = validate_gemm_backend(backend) if backend is not None else default_backend()
    if backend != "torch":
        reason = sample_contract_reason(x, weight, temperatures)
        if reason is None:
            return gemm_sample(x, weight, temperatures, seed, offset, logits_dtype)
        if backend == "hip":
            raise RuntimeError(f"HIP GEMM backend is unavailable: {reason}")
    return torch_sampler(_torch_logits(x, weight, logits_dtype), temperatures), None
