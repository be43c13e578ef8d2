"""ctypes binding of libnanovllm_gemm.so (declared in include/nanovllm_gemm.h).

The loader mirrors the reference's ``load_cuda_ops``
(nanovllm/kernels/_extension.py:36-68) in spirit: one cached load of a
prebuilt native module.  There is no JIT fallback and no pure-Python
substitute: when the library is missing, every entry point raises
``GemmLibraryError`` so a GPU run can never silently take another path.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libnanovllm_gemm.so"

# dtype and layout codes (values fixed by the C header)
F32, F16, BF16 = 0, 1, 2
B_NK, B_KN = 0, 1

# kernel ids (values fixed by the C header)
KERNEL_FP32_NAIVE = 0
KERNEL_FP32_TILED = 1
KERNEL_MFMA_DIRECT = 2
KERNEL_MFMA_STAGED = 3
KERNEL_SPLITK_DECODE = 4
KERNEL_GEMV_DECODE = 5
KERNEL_COUNT = 6

OK, EINVAL, EUNSUPPORTED, ELAUNCH = 0, -1, -2, -3

# Every function the header declares, with its ctypes signature.
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_VP = ctypes.c_void_p
_F32 = ctypes.c_float
_U64 = ctypes.c_uint64
SIGNATURES = {
    "nanovllm_gemm": (_INT, [_VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _VP]),
    "nanovllm_gemm_with_kernel": (_INT, [_INT, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _INT,
                                         _VP]),
    "nanovllm_gemm_select": (_INT, [_I64, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT]),
    "nanovllm_gemm_kernel_supports": (_INT, [_INT, _I64, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT]),
    "nanovllm_gemm_silu_mul": (_INT, [_VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _VP]),
    "nanovllm_gemm_silu_mul_with_kernel": (_INT, [_INT, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _INT,
                                                  _INT, _VP]),
    "nanovllm_gemm_silu_mul_select": (_INT, [_I64, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _INT]),
    "nanovllm_gemm_argmax": (_INT, [_VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _VP, _I64, _VP]),
    "nanovllm_gemm_argmax_noalloc": (_INT, [_VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _VP]),
    "nanovllm_gemm_argmax_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _INT]),
    "nanovllm_gemm_argmax_with_kernel": (_INT, [_INT, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _INT, _INT,
                                                _VP, _I64, _VP]),
    "nanovllm_gemm_argmax_select": (_INT, [_I64, _I64, _I64, _I64, _I64, _INT, _INT]),
    "nanovllm_gemm_sample": (_INT, [_VP, _VP, _VP, _U64, _U64, _VP, _VP, _I64, _I64, _I64, _I64, _I64, _INT, _INT,
                                    _VP, _I64, _VP]),
    "nanovllm_gemm_sample_with_kernel": (_INT, [_INT, _VP, _VP, _VP, _U64, _U64, _VP, _VP, _I64, _I64, _I64, _I64,
                                                _I64, _INT, _INT, _VP, _I64, _VP]),
    "nanovllm_gemm_gated": (_INT, [_VP, _VP, _VP, _VP] + [_I64] * 9 + [_INT, _INT, _VP, _I64, _VP]),
    "nanovllm_gemm_gated_workspace_bytes": (_I64, [_I64, _I64, _I64, _INT]),
    "nanovllm_gemm_gated_with_kernel": (_INT, [_INT, _VP, _VP, _VP, _VP] + [_I64] * 9 + [_INT, _INT, _VP, _I64, _VP]),
    "nanovllm_sigmoid_gate": (_INT, [_VP, _VP, _VP] + [_I64] * 7 + [_INT, _VP]),
    "nanovllm_gemm_add_rmsnorm": (_INT, [_VP, _VP, _VP, _F32, _VP, _VP, _VP] + [_I64] * 8
                                  + [_INT, _INT, _INT, _VP, _I64, _VP]),
    "nanovllm_gemm_add_rmsnorm_workspace_bytes": (_I64, [_I64, _I64, _INT]),
    "nanovllm_gemm_add_rmsnorm_with_kernel": (_INT, [_INT, _VP, _VP, _VP, _F32, _VP, _VP, _VP] + [_I64] * 8
                                              + [_INT, _INT, _INT, _VP, _I64, _VP]),
    "nanovllm_gemm_kernel_name": (ctypes.c_char_p, [_INT]),
    "nanovllm_gemm_last_error": (ctypes.c_char_p, []),
    "nanovllm_gemm_version": (_INT, []),
}


class GemmLibraryError(RuntimeError):
    """The native GEMM library is missing, failed to load, or returned an error."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    override = os.environ.get("NANOVLLM_GEMM_LIB")
    return Path(override) if override else LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not path.is_file():
            raise GemmLibraryError(
                f"{path.name} is not built (looked in {path.parent}); run __graft_entry__.build() "
                "or python inference-systems_amd/build.py"
            )
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as exc:  # pragma: no cover - depends on the host
            raise GemmLibraryError(f"failed to load {path}: {exc}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def is_available() -> bool:
    try:
        load()
    except GemmLibraryError:
        return False
    return True


def last_error() -> str:
    return load().nanovllm_gemm_last_error().decode()


def kernel_name(kernel_id: int) -> str:
    return load().nanovllm_gemm_kernel_name(kernel_id).decode()


def check(rc: int, what: str) -> None:
    if rc != OK:
        raise GemmLibraryError(f"{what} failed (code {rc}): {last_error()}")


def select(m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out, aligned16=True) -> int:
    """Kernel id the shape-selection table picks (negative code if invalid)."""
    return load().nanovllm_gemm_select(m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out, int(bool(aligned16)))


def kernel_supports(kernel_id, m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out, aligned16=True) -> bool:
    return bool(load().nanovllm_gemm_kernel_supports(kernel_id, m, n, k, lda, ldb, ldc, b_layout, dtype_in,
                                                     dtype_out, int(bool(aligned16))))


def silu_mul_select(m, n, k, lda, ldw, ldc, dtype_in, dtype_out, aligned16=True) -> int:
    """Kernel id of the fused gate/up + SiLU-and-mul (negative code if invalid)."""
    return load().nanovllm_gemm_silu_mul_select(m, n, k, lda, ldw, ldc, dtype_in, dtype_out, int(bool(aligned16)))


def silu_mul_raw(a_ptr, w_ptr, c_ptr, m, n, k, lda, ldw, ldc, dtype_in, dtype_out, stream,
                 kernel: int | None = None) -> None:
    """Enqueue one fused gate/up + SiLU-and-mul on `stream`; raise on error."""
    lib = load()
    if kernel is None:
        rc = lib.nanovllm_gemm_silu_mul(a_ptr, w_ptr, c_ptr, m, n, k, lda, ldw, ldc, dtype_in, dtype_out, stream)
    else:
        rc = lib.nanovllm_gemm_silu_mul_with_kernel(kernel, a_ptr, w_ptr, c_ptr, m, n, k, lda, ldw, ldc, dtype_in,
                                                    dtype_out, stream)
    check(rc, "nanovllm_gemm_silu_mul")


def argmax_workspace_bytes(m, n, k, lda, ldw, dtype_in) -> int:
    """Workspace bytes of the greedy head (negative code if invalid)."""
    return load().nanovllm_gemm_argmax_workspace_bytes(m, n, k, lda, ldw, dtype_in)


def argmax_select(m, n, k, lda, ldw, dtype_in, aligned16=True) -> int:
    return load().nanovllm_gemm_argmax_select(m, n, k, lda, ldw, dtype_in, int(bool(aligned16)))


def argmax_raw(a_ptr, w_ptr, tokens_ptr, logits_ptr, m, n, k, lda, ldw, dtype_in, logit_dtype, ws_ptr, ws_bytes,
               stream, kernel: int | None = None) -> None:
    """Enqueue the greedy LM head (GEMM pass + reduction) on `stream`; raise
    on error.  logit_dtype: ``dtype_in`` ranks the logits rounded to the
    input type (the reference's bf16 F.linear logits), ``F32`` the fp32 sums."""
    lib = load()
    if kernel is None:
        rc = lib.nanovllm_gemm_argmax(a_ptr, w_ptr, tokens_ptr, logits_ptr, m, n, k, lda, ldw, dtype_in, logit_dtype,
                                      ws_ptr, ws_bytes, stream)
    else:
        rc = lib.nanovllm_gemm_argmax_with_kernel(kernel, a_ptr, w_ptr, tokens_ptr, logits_ptr, m, n, k, lda, ldw,
                                                  dtype_in, logit_dtype, ws_ptr, ws_bytes, stream)
    check(rc, "nanovllm_gemm_argmax")


def sample_raw(a_ptr, w_ptr, t_ptr, seed, offset, tokens_ptr, scores_ptr, m, n, k, lda, ldw, dtype_in, logit_dtype,
               ws_ptr, ws_bytes, stream, kernel: int | None = None) -> None:
    """Enqueue the sampled LM head (GEMM pass + reduction) on `stream`; raise on error."""
    lib = load()
    seed &= (1 << 64) - 1
    offset &= (1 << 64) - 1
    if kernel is None:
        rc = lib.nanovllm_gemm_sample(a_ptr, w_ptr, t_ptr, seed, offset, tokens_ptr, scores_ptr, m, n, k, lda, ldw,
                                      dtype_in, logit_dtype, ws_ptr, ws_bytes, stream)
    else:
        rc = lib.nanovllm_gemm_sample_with_kernel(kernel, a_ptr, w_ptr, t_ptr, seed, offset, tokens_ptr, scores_ptr,
                                                  m, n, k, lda, ldw, dtype_in, logit_dtype, ws_ptr, ws_bytes, stream)
    check(rc, "nanovllm_gemm_sample")


def gemm_raw(a_ptr, b_ptr, c_ptr, m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out, stream,
             kernel: int | None = None) -> None:
    """Enqueue one GEMM on `stream` through the C ABI; raise on error."""
    lib = load()
    if kernel is None:
        rc = lib.nanovllm_gemm(a_ptr, b_ptr, c_ptr, m, n, k, lda, ldb, ldc, b_layout, dtype_in, dtype_out, stream)
    else:
        rc = lib.nanovllm_gemm_with_kernel(kernel, a_ptr, b_ptr, c_ptr, m, n, k, lda, ldb, ldc, b_layout, dtype_in,
                                           dtype_out, stream)
    check(rc, "nanovllm_gemm")


def gated_workspace_bytes(m, k, group, dtype_in) -> int:
    """Workspace bytes of the gated GEMM (0 when the gate is fused; negative code if invalid)."""
    return load().nanovllm_gemm_gated_workspace_bytes(m, k, group, dtype_in)


def gated_raw(a_ptr, gate_ptr, w_ptr, c_ptr, m, n, k, lda, ldg, group, group_stride, ldw, ldc, dtype_in, dtype_out,
              ws_ptr, ws_bytes, stream, kernel: int | None = None) -> None:
    """Enqueue the gated-attention output projection on `stream`; raise on error."""
    lib = load()
    args = (a_ptr, gate_ptr, w_ptr, c_ptr, m, n, k, lda, ldg, group, group_stride, ldw, ldc, dtype_in, dtype_out,
            ws_ptr, ws_bytes, stream)
    rc = lib.nanovllm_gemm_gated(*args) if kernel is None else lib.nanovllm_gemm_gated_with_kernel(kernel, *args)
    check(rc, "nanovllm_gemm_gated")


def sigmoid_gate_raw(a_ptr, gate_ptr, out_ptr, m, k, lda, ldg, group, group_stride, ldo, dtype, stream) -> None:
    """Enqueue the standalone output gate on `stream`; raise on error."""
    check(load().nanovllm_sigmoid_gate(a_ptr, gate_ptr, out_ptr, m, k, lda, ldg, group, group_stride, ldo, dtype,
                                       stream), "nanovllm_sigmoid_gate")


def add_rmsnorm_workspace_bytes(m, k, dtype_in) -> int:
    """Workspace bytes of the add + RMSNorm GEMM (0 for m <= 32; negative code if invalid)."""
    return load().nanovllm_gemm_add_rmsnorm_workspace_bytes(m, k, dtype_in)


def add_rmsnorm_raw(h_ptr, r_ptr, nw_ptr, eps, w_ptr, c_ptr, res_ptr, m, n, k, ldh, ldr, ldw, ldc, ldres, silu_mul,
                    dtype_in, dtype_out, ws_ptr, ws_bytes, stream, kernel: int | None = None) -> None:
    """Enqueue the residual add + RMSNorm + projection on `stream`; raise on error."""
    lib = load()
    args = (h_ptr, r_ptr, nw_ptr, eps, w_ptr, c_ptr, res_ptr, m, n, k, ldh, ldr, ldw, ldc, ldres, int(silu_mul),
            dtype_in, dtype_out, ws_ptr, ws_bytes, stream)
    rc = (lib.nanovllm_gemm_add_rmsnorm(*args) if kernel is None
          else lib.nanovllm_gemm_add_rmsnorm_with_kernel(kernel, *args))
    check(rc, "nanovllm_gemm_add_rmsnorm")
