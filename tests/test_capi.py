"""CPU tests of the C ABI: the library loads, exports every symbol the header
declares, validates arguments before touching the GPU, and its shape-selection
table maps every valid problem to a kernel of its own (the replacement for
supports_wmma / choose_path, cuda_kernels/gemm/src/gemm_bench.cu:252-273).
No test here launches a kernel."""
from __future__ import annotations

import itertools
import re
from pathlib import Path

import pytest

from conftest import PKG, ROOT

L = PKG._lib
F32, F16, BF16 = L.F32, L.F16, L.BF16
NK, KN = L.B_NK, L.B_KN


def _declared_functions():
    names = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = header.read_text()
        names += re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(nanovllm_\w+)\s*\(", text, flags=re.M)
    return names


def test_every_declared_symbol_is_exported(lib):
    names = _declared_functions()
    assert len(names) >= 7
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(L.SIGNATURES), "ctypes signatures must cover exactly the header"


def test_version_and_names(lib):
    assert lib.nanovllm_gemm_version() >> 16 == 2
    expected = ["fp32_naive", "fp32_tiled", "mfma_direct", "mfma_staged", "splitk_decode", "gemv_decode"]
    assert [L.kernel_name(i) for i in range(L.KERNEL_COUNT)] == expected
    assert L.kernel_name(99) == "unknown" and L.kernel_name(-1) == "unknown"


@pytest.mark.parametrize("args,code,msg", [
    (dict(m=4, n=4, k=0), L.EINVAL, "k must be positive"),
    (dict(m=-1, n=4, k=4), L.EINVAL, "non-negative"),
    (dict(m=4, n=4, k=8, lda=7), L.EINVAL, "lda"),
    (dict(m=4, n=4, k=8, ldb=7), L.EINVAL, "ldb"),
    (dict(m=4, n=9, k=8, ldb=8, layout=KN), L.EINVAL, "ldb"),
    (dict(m=4, n=9, k=8, ldc=8), L.EINVAL, "ldc"),
    (dict(m=4, n=4, k=8, layout=2), L.EINVAL, "b_layout"),
    (dict(m=4, n=4, k=8, din=F32, dout=BF16), L.EUNSUPPORTED, "dtype pair"),
    (dict(m=4, n=4, k=8, din=BF16, dout=F16), L.EUNSUPPORTED, "dtype pair"),
    (dict(m=4, n=4, k=8, din=7, dout=F32), L.EINVAL, "dtype code"),
])
def test_select_rejects_invalid_problems(args, code, msg):
    m, n, k = args["m"], args["n"], args["k"]
    layout = args.get("layout", NK)
    lda = args.get("lda", k)
    ldb = args.get("ldb", k if layout == NK else n)
    ldc = args.get("ldc", n)
    rc = L.select(m, n, k, lda, ldb, ldc, layout, args.get("din", BF16), args.get("dout", BF16))
    assert rc == code
    assert msg in L.last_error()


def test_gemm_validates_before_launch(lib):
    # Invalid sizes and null pointers are rejected on the host: no GPU needed.
    rc = lib.nanovllm_gemm(None, None, None, 4, 4, 0, 4, 4, 4, NK, BF16, BF16, None)
    assert rc == L.EINVAL and "k must be positive" in L.last_error()
    rc = lib.nanovllm_gemm(None, None, None, 4, 4, 8, 8, 8, 4, NK, BF16, BF16, None)
    assert rc == L.EINVAL and "non-null" in L.last_error()
    # Empty output: a valid no-op that never dereferences the pointers.
    assert lib.nanovllm_gemm(None, None, None, 0, 4, 8, 8, 8, 4, NK, BF16, BF16, None) == L.OK
    assert lib.nanovllm_gemm(None, None, None, 4, 0, 8, 8, 8, 1, NK, BF16, BF16, None) == L.OK
    assert L.last_error() == ""
    rc = lib.nanovllm_gemm_with_kernel(-3, None, None, None, 4, 4, 8, 8, 8, 4, NK, BF16, BF16, None)
    assert rc == L.EINVAL and "kernel id" in L.last_error()
    rc = lib.nanovllm_gemm_with_kernel(17, None, None, None, 4, 4, 8, 8, 8, 4, NK, BF16, BF16, None)
    assert rc == L.EINVAL


def test_gemm_with_kernel_refuses_unsupported_rung(lib):
    # fp32_tiled cannot take bf16; splitk_decode cannot take M = 65, nor
    # M = 33 with 65536 W rows; the check happens before any launch (pointers
    # are dummies never dereferenced).
    dummy = 1 << 20
    rc = lib.nanovllm_gemm_with_kernel(L.KERNEL_FP32_TILED, dummy, dummy, dummy, 4, 4, 8, 8, 8, 4, NK, BF16, BF16,
                                       None)
    assert rc == L.EUNSUPPORTED and "fp32_tiled" in L.last_error()
    rc = lib.nanovllm_gemm_with_kernel(L.KERNEL_SPLITK_DECODE, dummy, dummy, dummy, 65, 64, 64, 64, 64, 64, NK,
                                       BF16, BF16, None)
    assert rc == L.EUNSUPPORTED
    rc = lib.nanovllm_gemm_with_kernel(L.KERNEL_SPLITK_DECODE, dummy, dummy, dummy, 33, 65536, 64, 64, 64, 65536,
                                       NK, BF16, BF16, None)
    assert rc == L.EUNSUPPORTED
    assert L.kernel_supports(L.KERNEL_SPLITK_DECODE, 64, 65535, 64, 64, 64, 65535, NK, BF16, BF16, 1)
    assert L.kernel_supports(L.KERNEL_SPLITK_DECODE, 32, 151936, 64, 64, 64, 151936, NK, BF16, BF16, 1)


def _expected(m, n, k, lda, ldb, layout, din, aligned):
    if din == F32:
        return L.KERNEL_FP32_TILED
    vec = aligned and k % 8 == 0 and lda % 8 == 0 and ldb % 8 == 0 and layout == NK
    if vec:
        if m == 1 and n * k * 2 <= 64 * 2 ** 20:
            return L.KERNEL_GEMV_DECODE
        if m <= 32:
            return L.KERNEL_SPLITK_DECODE
        # 33 <= M <= 64: narrow problems stream W on splitk_decode as well
        if m <= 64 and (n <= 4096 or (n <= 10240 and k <= 1024)):
            return L.KERNEL_SPLITK_DECODE
        return L.KERNEL_MFMA_STAGED
    # B[K,N] with whole 8-column chunks: splitk_decode up to M = 32, and up to
    # M = 64 on at most 4096 columns; the staged kernel above
    kn_vec = aligned and k % 8 == 0 and lda % 8 == 0 and ldb % 8 == 0 and n % 8 == 0 and layout == KN
    if kn_vec:
        return L.KERNEL_SPLITK_DECODE if m <= 32 or (m <= 64 and n <= 4096) else L.KERNEL_MFMA_STAGED
    return L.KERNEL_MFMA_DIRECT


PAIRS = [(F32, F32), (F16, F16), (F16, F32), (BF16, BF16), (BF16, F32)]


@pytest.mark.parametrize("din,dout", PAIRS)
def test_selection_table_total_and_self_consistent(din, dout):
    """Every valid problem maps to one of this library's kernels, that kernel
    supports it, and the table follows its stated rule."""
    ms = [0, 1, 4, 16, 31, 32, 33, 48, 64, 65, 127, 2048]
    ns = [1, 15, 193, 4096, 4097, 8224, 10240, 10241, 151936]
    ks = [1, 7, 8, 65, 1024, 1032, 3584]
    for m, n, k, layout, aligned, pad in itertools.product(ms, ns, ks, (NK, KN), (0, 1), (0, 3)):
        lda = k + pad
        ldb = (k if layout == NK else n) + pad
        kid = L.select(m, n, k, lda, ldb, n, layout, din, dout, aligned)
        assert 0 <= kid < L.KERNEL_COUNT
        assert kid == _expected(m, n, k, lda, ldb, layout, din, aligned), (m, n, k, layout, aligned, pad)
        assert L.kernel_supports(kid, m, n, k, lda, ldb, n, layout, din, dout, aligned)


def test_selection_on_workloads_and_qwen_shapes():
    W = PKG.workloads
    code = {"torch.float32": F32, "torch.float16": F16, "torch.bfloat16": BF16}
    want = {
        "fp32_square_1024": {1024: "fp32_tiled"},
        "bf16_prefill_2048x4096x1024": {2048: "mfma_staged"},
        "bf16_decode_n6144_k1024": {1: "gemv_decode", 4: "splitk_decode", 8: "splitk_decode",
                                    16: "splitk_decode", 32: "splitk_decode"},
        "fp16_down_4096x1024x3584": {4096: "mfma_staged"},
        "bf16_lm_head_n151936_k1024": {1: "splitk_decode", 32: "splitk_decode", 512: "mfma_staged"},
    }
    for name, wl in W.WORKLOADS.items():
        for m in wl.ms:
            ldb = wl.k if wl.b_layout == NK else wl.n
            kid = L.select(m, wl.n, wl.k, wl.k, ldb, wl.n, wl.b_layout, code[str(wl.dtype_in)],
                           code[str(wl.dtype_out)], 1)
            assert L.kernel_name(kid) == want[name][m], (name, m)
    for label, m, n, k in W.QWEN35_SHAPES:
        kid = L.select(m, n, k, k, k, n, NK, BF16, BF16, 1)
        want_k = "gemv_decode" if m == 1 else ("splitk_decode" if m <= 64 else "mfma_staged")
        assert L.kernel_name(kid) == want_k, label
        # the reference's B[K,N] layout of the same shapes: splitk_decode up to M = 32 (and
        # M = 64 on N <= 4096), the staged rung above
        kid = L.select(m, n, k, k, n, n, KN, BF16, F32, 1)
        want_kn = "splitk_decode" if m <= 32 or (m <= 64 and n <= 4096) else "mfma_staged"
        assert L.kernel_name(kid) == want_kn, label


def test_no_vendor_kernel_id():
    # The reference falls back to cuBLAS outside a narrow regime
    # (gemm_bench.cu:260-273); here every id is one of the ladder's kernels.
    names = {L.kernel_name(i) for i in range(L.KERNEL_COUNT)}
    assert not any("blas" in nm for nm in names)


# ---------------------------------------------------------------------------
# Fused gate/up projection + SiLU-and-mul
# ---------------------------------------------------------------------------
def _expected_silu(m, n, k, lda, ldw, aligned):
    if not (aligned and k % 8 == 0 and lda % 8 == 0 and ldw % 8 == 0):
        return L.EUNSUPPORTED
    if m <= 32 or (m <= 64 and 2 * n <= 16384):
        return L.KERNEL_SPLITK_DECODE
    return L.KERNEL_MFMA_STAGED


@pytest.mark.parametrize("din,dout", [(F16, F16), (F16, F32), (BF16, BF16), (BF16, F32)])
def test_silu_mul_selection(din, dout):
    for m, n, k, aligned, pad in itertools.product([1, 2, 32, 33, 64, 65, 2048], [1, 100, 3584, 8192, 8193, 75968],
                                                   [8, 72, 1024, 1000, 7], (0, 1), (0, 2)):
        lda, ldw = k + pad, k + pad
        got = L.silu_mul_select(m, n, k, lda, ldw, n, din, dout, aligned)
        assert got == _expected_silu(m, n, k, lda, ldw, aligned), (m, n, k, aligned, pad)
        if got == L.EUNSUPPORTED:
            assert "16-byte aligned" in L.last_error()


@pytest.mark.parametrize("args,code,msg", [
    (dict(din=F32, dout=F32), L.EUNSUPPORTED, "silu_mul"),
    (dict(din=BF16, dout=F16), L.EUNSUPPORTED, "silu_mul"),
    (dict(k=0), L.EINVAL, "k must be positive"),
    (dict(ldw=4), L.EINVAL, "ldw"),
    (dict(ldc=3), L.EINVAL, "ldc"),
    (dict(m=-1), L.EINVAL, "non-negative"),
])
def test_silu_mul_rejects_invalid(args, code, msg):
    m, n, k = args.get("m", 4), args.get("n", 8), args.get("k", 16)
    rc = L.silu_mul_select(m, n, k, args.get("lda", k), args.get("ldw", k), args.get("ldc", n),
                           args.get("din", BF16), args.get("dout", BF16))
    assert rc == code and msg in L.last_error()


def test_silu_mul_validates_before_launch(lib):
    assert lib.nanovllm_gemm_silu_mul(None, None, None, 0, 8, 16, 16, 16, 8, BF16, BF16, None) == L.OK
    rc = lib.nanovllm_gemm_silu_mul(None, None, None, 4, 8, 16, 16, 16, 8, BF16, BF16, None)
    assert rc == L.EINVAL and "non-null" in L.last_error()
    dummy = 1 << 20
    rc = lib.nanovllm_gemm_silu_mul_with_kernel(L.KERNEL_MFMA_DIRECT, dummy, dummy, dummy, 4, 8, 16, 16, 16, 8,
                                                BF16, BF16, None)
    assert rc == L.EUNSUPPORTED and "mfma_direct" in L.last_error()
    rc = lib.nanovllm_gemm_silu_mul_with_kernel(L.KERNEL_GEMV_DECODE, dummy, dummy, dummy, 4, 8, 16, 16, 16, 8,
                                                BF16, BF16, None)
    assert rc == L.EUNSUPPORTED
    rc = lib.nanovllm_gemm_silu_mul_with_kernel(99, dummy, dummy, dummy, 4, 8, 16, 16, 16, 8, BF16, BF16, None)
    assert rc == L.EINVAL and "kernel id" in L.last_error()
    # unaligned pointers: only the vector path exists for the fused op
    rc = lib.nanovllm_gemm_silu_mul(dummy + 2, dummy, dummy, 4, 8, 16, 16, 16, 8, BF16, BF16, None)
    assert rc == L.EUNSUPPORTED and "aligned" in L.last_error()


# ---------------------------------------------------------------------------
# Greedy LM head (argmax without logits)
# ---------------------------------------------------------------------------
def test_argmax_workspace_and_selection():
    for m, n in itertools.product([1, 7, 32, 33, 512], [1, 15, 16, 17, 151936]):
        cols = 16 if m <= 32 else 128
        assert L.argmax_workspace_bytes(m, n, 1024, 1024, 1024, BF16) == -(-n // cols) * m * 8
        want = L.KERNEL_SPLITK_DECODE if m <= 32 else L.KERNEL_MFMA_STAGED
        assert L.argmax_select(m, n, 1024, 1024, 1024, BF16, True) == want
        assert L.argmax_select(m, n, 1024, 1024, 1024, F16, False) == L.EUNSUPPORTED
    assert L.argmax_select(4, 100, 1000 + 4, 1004, 1004, BF16, True) == L.EUNSUPPORTED   # k % 8 != 0


@pytest.mark.parametrize("args,code,msg", [
    (dict(din=F32), L.EUNSUPPORTED, "float16 or bfloat16"),
    (dict(din=9), L.EINVAL, "float16 or bfloat16"),
    (dict(n=0), L.EINVAL, "n must be in"),
    (dict(n=2 ** 32), L.EINVAL, "n must be in"),
    (dict(k=0), L.EINVAL, "k must be positive"),
    (dict(ldw=8), L.EINVAL, "ldw"),
    (dict(m=-2), L.EINVAL, "non-negative"),
])
def test_argmax_rejects_invalid(args, code, msg):
    m, n, k = args.get("m", 4), args.get("n", 64), args.get("k", 16)
    rc = L.argmax_workspace_bytes(m, n, k, args.get("lda", k), args.get("ldw", k), args.get("din", BF16))
    assert rc == code and msg in L.last_error()


def test_argmax_validates_before_launch(lib):
    assert lib.nanovllm_gemm_argmax(None, None, None, None, 0, 64, 16, 16, 16, BF16, BF16, None, 0, None) == L.OK
    rc = lib.nanovllm_gemm_argmax(None, None, None, None, 4, 64, 16, 16, 16, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "non-null" in L.last_error()
    dummy = 1 << 20
    need = L.argmax_workspace_bytes(4, 64, 16, 16, 16, BF16)
    rc = lib.nanovllm_gemm_argmax(dummy, dummy, dummy, None, 4, 64, 16, 16, 16, BF16, BF16, dummy, need - 8, None)
    assert rc == L.EINVAL and f"needs {need}" in L.last_error()
    rc = lib.nanovllm_gemm_argmax(dummy, dummy, dummy, None, 4, 64, 16, 16, 16, BF16, BF16, dummy + 4, need, None)
    assert rc == L.EINVAL and "8-byte aligned" in L.last_error()
    rc = lib.nanovllm_gemm_argmax_with_kernel(L.KERNEL_GEMV_DECODE, dummy, dummy, dummy, None, 4, 64, 16, 16, 16,
                                              BF16, F32, dummy, need, None)
    assert rc == L.EUNSUPPORTED and "gemv_decode" in L.last_error()
    rc = lib.nanovllm_gemm_argmax_with_kernel(L.KERNEL_SPLITK_DECODE, dummy, dummy, dummy, None, 33, 64, 16, 16, 16,
                                              BF16, BF16, dummy, 10 ** 6, None)
    assert rc == L.EUNSUPPORTED


@pytest.mark.parametrize("din,logit,ok", [(BF16, BF16, True), (BF16, F32, True), (BF16, F16, False),
                                          (F16, F16, True), (F16, F32, True), (F16, BF16, False), (BF16, 7, False)])
def test_argmax_logit_dtype(lib, din, logit, ok):
    """The LM head ranks the logits rounded to the input type (the
    reference's F.linear output) or the fp32 sums; any other ranking type is
    rejected before anything is launched (m = 0 launches nothing when valid)."""
    rc = lib.nanovllm_gemm_argmax(None, None, None, None, 0, 64, 16, 16, 16, din, logit, None, 0, None)
    rc_s = lib.nanovllm_gemm_sample(None, None, None, 1, 2, None, None, 0, 64, 16, 16, 16, din, logit, None, 0, None)
    if ok:
        assert rc == L.OK and rc_s == L.OK
    else:
        assert rc == L.EINVAL and "logit_dtype" in L.last_error()
        assert rc_s == L.EINVAL


def test_argmax_noalloc_validates_before_launch(lib):
    """The no-allocation greedy head: the argmax checks, then the bound of
    its 8 MiB scratch, all before any device call (m = 0 returns at once)."""
    assert lib.nanovllm_gemm_argmax_noalloc(None, None, None, None, 0, 64, 16, 16, 16, BF16, BF16, None) == L.OK
    rc = lib.nanovllm_gemm_argmax_noalloc(None, None, None, None, 4, 64, 16, 16, 16, L.F32, F32, None)
    assert rc == L.EUNSUPPORTED
    rc = lib.nanovllm_gemm_argmax_noalloc(None, None, None, None, 4, 64, 16, 16, 16, BF16, F16, None)
    assert rc == L.EINVAL and "logit_dtype" in L.last_error()
    # The Qwen vocabulary: 1187 keys of 8 bytes per row (128 columns per key),
    # so the 8 MiB array holds m <= 883; m = 884 is refused before any device call.
    assert L.argmax_workspace_bytes(883, 151936, 1024, 1024, 1024, BF16) <= 8 << 20
    assert L.argmax_workspace_bytes(884, 151936, 1024, 1024, 1024, BF16) > 8 << 20
    for m in (884, 1024):
        rc = lib.nanovllm_gemm_argmax_noalloc(None, None, None, None, m, 151936, 1024, 1024, 1024, BF16, BF16, None)
        assert rc == L.EINVAL and "scratch" in L.last_error() and "nanovllm_gemm_argmax" in L.last_error()


def test_sample_validates_before_launch(lib):
    """The sampled head shares the greedy head's checks and adds its own:
    temperatures must be a non-null, 4-byte aligned device pointer."""
    assert lib.nanovllm_gemm_sample(None, None, None, 1, 2, None, None, 0, 64, 16, 16, 16, BF16, BF16, None, 0,
                                    None) == L.OK
    dummy = 1 << 20
    need = L.argmax_workspace_bytes(4, 64, 16, 16, 16, BF16)
    rc = lib.nanovllm_gemm_sample(dummy, dummy, None, 1, 2, dummy, None, 4, 64, 16, 16, 16, BF16, BF16, dummy, need,
                                  None)
    assert rc == L.EINVAL and "temperatures" in L.last_error()
    rc = lib.nanovllm_gemm_sample(dummy, dummy, dummy + 2, 1, 2, dummy, None, 4, 64, 16, 16, 16, BF16, BF16, dummy,
                                  need, None)
    assert rc == L.EINVAL and "4-byte aligned" in L.last_error()
    rc = lib.nanovllm_gemm_sample(dummy, dummy, dummy, 1, 2, dummy, None, 4, 64, 16, 16, 16, L.F32, L.F32, dummy,
                                  need, None)
    assert rc == L.EUNSUPPORTED
    rc = lib.nanovllm_gemm_sample_with_kernel(L.KERNEL_FP32_TILED, dummy, dummy, dummy, 1, 2, dummy, None, 4, 64,
                                              16, 16, 16, BF16, BF16, dummy, need, None)
    assert rc == L.EUNSUPPORTED and "fp32_tiled" in L.last_error()
    rc = lib.nanovllm_gemm_sample_with_kernel(99, dummy, dummy, dummy, 1, 2, dummy, None, 4, 64, 16, 16, 16, BF16,
                                              BF16, dummy, need, None)
    assert rc == L.EINVAL and "unknown kernel" in L.last_error()


# ---------------------------------------------------------------------------
# GEMMs with a prologue (output gate, residual add + RMSNorm)
# ---------------------------------------------------------------------------
def test_prologue_workspace_bytes():
    # enough for any kernel: the gated operand (M x K elements), plus for the
    # norm the fp32 row scales, each rounded up to 256 bytes
    assert L.gated_workspace_bytes(32, 2048, 256, BF16) == 32 * 2048 * 2
    assert L.gated_workspace_bytes(4, 160, 40, BF16) == 1280
    assert L.gated_workspace_bytes(4, 100, 40, BF16) == L.EINVAL      # group does not divide K
    assert L.gated_workspace_bytes(4, 128, 64, F32) == L.EUNSUPPORTED
    assert L.add_rmsnorm_workspace_bytes(32, 1024, BF16) == 32 * 2048 + 256
    assert L.add_rmsnorm_workspace_bytes(33, 1000, BF16) == (33 * 2000 + 255) // 256 * 256 + 256
    assert L.add_rmsnorm_workspace_bytes(33, 1000, F16) == L.EUNSUPPORTED
    assert L.add_rmsnorm_workspace_bytes(-1, 1024, BF16) == L.EINVAL


def test_gated_validates_before_launch(lib):
    d = 1 << 20
    call = lambda *a: lib.nanovllm_gemm_gated(*a)  # noqa: E731
    # m = 0 is a no-op even with null pointers
    assert call(None, None, None, None, 0, 64, 512, 512, 1024, 256, 512, 512, 64, BF16, BF16, None, 0, None) == L.OK
    rc = call(None, None, None, None, 4, 64, 512, 512, 1024, 256, 512, 512, 64, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "non-null" in L.last_error()
    rc = call(d, d, d, d, 4, 64, 512, 512, 1024, 200, 512, 512, 64, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "divide" in L.last_error()
    rc = call(d, d, d, d, 4, 64, 512, 512, 1024, 256, 128, 512, 64, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "group_stride" in L.last_error()
    rc = call(d, d, d, d, 4, 64, 512, 512, 700, 256, 512, 512, 64, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "ldg" in L.last_error()
    rc = call(d, d + 2, d, d, 4, 64, 512, 512, 1024, 256, 512, 512, 64, BF16, BF16, None, 0, None)
    assert rc == L.EUNSUPPORTED and "aligned" in L.last_error()
    rc = call(d, d, d, d, 4, 64, 512, 512, 1024, 256, 512, 512, 64, F32, F32, None, 0, None)
    assert rc == L.EUNSUPPORTED and "float16 or bfloat16" in L.last_error()
    # the fused path (M <= 32, head size a multiple of 64) takes no workspace
    assert L.gated_workspace_bytes(4, 512, 256, BF16) > 0
    # M > 32 needs the workspace
    rc = call(d, d, d, d, 40, 64, 512, 512, 1024, 256, 512, 512, 64, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "workspace" in L.last_error()
    # the fused gate cannot take a head size that is not a multiple of 64
    rc = lib.nanovllm_gemm_gated_with_kernel(L.KERNEL_SPLITK_DECODE, d, d, d, d, 4, 64, 480, 480, 960, 40, 80, 480,
                                             64, BF16, BF16, None, 0, None)
    assert rc == L.EUNSUPPORTED and "multiple of 64" in L.last_error()
    rc = lib.nanovllm_sigmoid_gate(d, d, d, 4, 512, 512, 1024, 256, 512, 100, BF16, None)
    assert rc == L.EINVAL and "ldo" in L.last_error()


def test_add_rmsnorm_validates_before_launch(lib):
    d = 1 << 20
    call = lambda *a: lib.nanovllm_gemm_add_rmsnorm(*a)  # noqa: E731
    assert call(None, None, None, 1e-6, None, None, None, 0, 64, 512, 512, 512, 512, 64, 512, 0, BF16, BF16,
                None, 0, None) == L.OK
    rc = call(None, None, None, 1e-6, None, None, None, 4, 64, 512, 512, 512, 512, 64, 512, 0, BF16, BF16, None, 0,
              None)
    assert rc == L.EINVAL and "non-null" in L.last_error()
    rc = call(d, d, d, -1.0, d, d, d, 4, 64, 512, 512, 512, 512, 64, 512, 0, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "eps" in L.last_error()
    rc = call(d, d, d, 1e-6, d, d, d, 4, 0, 512, 512, 512, 512, 64, 512, 0, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "n must be positive" in L.last_error()
    rc = call(d, d, d, 1e-6, d, d, d, 4, 64, 512, 500, 512, 512, 64, 512, 0, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "ldh" in L.last_error()
    rc = call(d, d, d, 1e-6, d, d, d + 8, 4, 64, 512, 512, 512, 512, 64, 512, 0, BF16, BF16, None, 0, None)
    assert rc == L.EUNSUPPORTED and "aligned" in L.last_error()
    rc = call(d, d, d, 1e-6, d, d, d, 4, 64, 512, 512, 512, 512, 64, 512, 0, BF16, F16, None, 0, None)
    assert rc == L.EUNSUPPORTED and "dtype" in L.last_error()
    # fp16 is refused: the unscaled operand s (1 + w) can leave its range
    rc = call(d, d, d, 1e-6, d, d, d, 4, 64, 512, 512, 512, 512, 64, 512, 0, F16, F16, None, 0, None)
    assert rc == L.EUNSUPPORTED and "bfloat16 inputs only" in L.last_error()
    rc = call(d, d, d, 1e-6, d, d, d, 40, 64, 512, 512, 512, 512, 64, 512, 0, BF16, BF16, None, 0, None)
    assert rc == L.EINVAL and "workspace" in L.last_error()
    rc = lib.nanovllm_gemm_add_rmsnorm_with_kernel(L.KERNEL_SPLITK_DECODE, d, d, d, 1e-6, d, d, d, 40, 64, 512,
                                                   512, 512, 512, 64, 512, 0, BF16, BF16, None, 0, None)
    assert rc == L.EUNSUPPORTED and "m <= 32" in L.last_error()
    rc = lib.nanovllm_gemm_add_rmsnorm_with_kernel(L.KERNEL_GEMV_DECODE, d, d, d, 1e-6, d, d, d, 40, 64, 512,
                                                   512, 512, 512, 64, 512, 0, BF16, BF16, None, 0, None)
    assert rc == L.EUNSUPPORTED and "gemv_decode" in L.last_error()
