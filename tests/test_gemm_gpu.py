"""GPU parity tests of the HIP kernels against the CPU oracle.

Bars (written out where they are applied):
  * known-answer inputs (gemm_bench.cu:296-305, gemm_wmma.cu:300-311) give an
    exact fp32 sum in any order, so every kernel must return the exact value
    rounded once to the output type: bit-exact, 0 ULP (the reference
    recorded max-abs 0 on all 20 WMMA rows, rtx3060_gemm_matrix.csv:4-23);
  * random bf16/fp16 inputs: every element within 2 ulp of the fp32-
    accumulated reference (the host's fp32 GEMM of the same rounded inputs)
    rounded once to the output type T, except cancellation elements
    (|R| <= 2^-6 sum_k |a w|, R the float64 product), of which at most
    oracle.cancellation_cap may exceed it (1 in 30000 bf16 outputs, 1 in 2000
    fp16 outputs, at least 8); and every element within
    2 ulp_T(R) + K 2^-24 sum_k |a w| of R;
  * FP32: relative Frobenius error <= 1e-5 against torch.matmul, and the
    reference's elementwise check 1e-4 + 1e-4 |ref| (common.cuh:18-31).
"""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

from conftest import PKG
from oracle import gemm_oracle as orc

pytestmark = pytest.mark.gpu

L = PKG._lib
W = PKG.workloads
G = importlib.import_module("inference_systems_amd.kernels.gemm")
DEV = torch.device("cuda:0")
NAME = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}
CODE = {torch.float32: L.F32, torch.float16: L.F16, torch.bfloat16: L.BF16}
LAYOUT = {L.B_NK: "nk", L.B_KN: "kn"}


def _say(msg):
    print(msg, flush=True)


def _to_np_out(t: torch.Tensor, dtype: torch.dtype):
    t = t.cpu()
    if dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _fp32_reference(a: torch.Tensor, b: torch.Tensor, layout: int, dout: torch.dtype, rows=None):
    """The fp32-accumulated CPU reference of the rounded inputs (torch's
    float32 GEMM on the host), rounded once to the output type and encoded
    like _to_np_out."""
    a32 = a.float() if rows is None else a.float()[rows]
    b32 = b.float()
    r32 = a32 @ (b32.T if layout == L.B_NK else b32)
    return _to_np_out(r32.to(dout), dout)


def _check_tolerance(got: torch.Tensor, a: torch.Tensor, b: torch.Tensor, layout: int, dout: torch.dtype,
                     rows=None):
    """Narrow outputs: every element within 2 ulp of the fp32-accumulated
    reference rounded once, except elements whose exact value lies within
    the fp32 accumulation bound of zero (oracle.narrow_parity: cancellation
    elements, |R| <= 2^-6 sum |a w|, at most oracle.cancellation_cap of them
    beyond it),
    and every element within 2 ulp of R plus that bound, R the float64
    product.
    fp32 outputs: the bound plus relative Frobenius <= 1e-5.  Returns the
    ULP statistics."""
    a64 = a.double().numpy()
    b64 = b.double().numpy()
    got_all = got
    if rows is not None:
        a64 = a64[rows]
        got = got[rows]
    lay = LAYOUT[layout]
    r = orc.gemm_f64(a64, b64, lay)
    s = orc.abs_products_f64(a64, b64, lay)
    k = a.shape[1]
    tol = orc.gemm_tolerance(r, s, k, NAME[dout])
    g64 = got.double().cpu().numpy()
    err = np.abs(g64 - r)
    bad = err > tol
    assert np.isfinite(g64).all(), "non-finite output"
    assert not bad.any(), f"{int(bad.sum())} elements outside tolerance; worst excess {float((err - tol).max()):.3g}"
    if dout == torch.float32:
        # fp32 logits: reordering K = 1024 products already moves an fp32 sum
        # by tens of fp32 ulps, so "2 ulp" is not a meaningful elementwise
        # bar; the bound above is, plus a normwise one.
        rel = orc.rel_frobenius(g64, r)
        assert rel <= 1e-5, f"relative Frobenius error {rel:.3g}"
        return {"rel_frobenius": rel}
    stats = orc.narrow_parity(_to_np_out(got, dout), _fp32_reference(a, b, layout, dout, rows), r, s, NAME[dout])
    _assert_narrow(stats, NAME[dout])
    del got_all
    return stats


def _assert_narrow(stats, dtype: str):
    """Every non-cancellation element within 2 ulp of the fp32 reference,
    and at most oracle.cancellation_cap cancellation elements beyond it."""
    ok = stats.pop("ok")
    _say(f"  narrow {dtype}: {ok.size} outputs, {stats['cancel_beyond']} cancellation elements beyond 2 ulp "
         f"(cap {orc.cancellation_cap(ok.size, dtype)}), max ulp {stats['max_ulp_checked']}")
    assert ok.all(), f"{int((~ok).sum())} elements beyond 2 ulp of the fp32 reference ({stats})"
    assert stats["cancel_beyond"] <= orc.cancellation_cap(ok.size, dtype), stats


# ---------------------------------------------------------------------------
# Every rung of the ladder on small and ragged shapes
# ---------------------------------------------------------------------------
SMALL_SHAPES = [(1, 1, 8), (5, 7, 9), (1, 37, 64), (16, 16, 16), (31, 65, 72), (33, 100, 136),
                (127, 193, 65), (130, 300, 264), (64, 1024, 2048), (257, 129, 520)]
KERNELS = [L.KERNEL_FP32_NAIVE, L.KERNEL_FP32_TILED, L.KERNEL_MFMA_DIRECT, L.KERNEL_MFMA_STAGED,
           L.KERNEL_SPLITK_DECODE, L.KERNEL_GEMV_DECODE]
PAIRS = [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
         (torch.float16, torch.float16), (torch.float16, torch.float32)]


def _ladder_cases():
    """Every rung with the dtype pairs and layouts it accepts: the FP32 rungs
    take fp32 only, the matrix-core rungs bf16 / fp16 only, and gemv_decode
    W[N,K] only."""
    for kernel in KERNELS:
        fp32_rung = kernel in (L.KERNEL_FP32_NAIVE, L.KERNEL_FP32_TILED)
        for din, dout in PAIRS:
            if fp32_rung != (din == torch.float32):
                continue
            for layout in (L.B_NK, L.B_KN):
                if kernel == L.KERNEL_GEMV_DECODE and layout == L.B_KN:
                    continue
                yield pytest.param(kernel, din, dout, layout,
                                   id=f"{LAYOUT[layout]}-{NAME[din]}-{NAME[dout]}-{L.kernel_name(kernel)}")


@pytest.mark.parametrize("kernel,din,dout,layout", list(_ladder_cases()))
def test_ladder_parity_small(kernel, din, dout, layout):
    gen = torch.Generator().manual_seed(11)
    ran = 0
    for m, n, k in SMALL_SHAPES:
        ldb = k if layout == L.B_NK else n
        if not L.kernel_supports(kernel, m, n, k, k, ldb, n, layout, CODE[din], CODE[dout], True):
            continue
        _say(f"ladder {L.kernel_name(kernel)} {NAME[din]}->{NAME[dout]} {LAYOUT[layout]} M={m} N={n} K={k}")
        a = torch.randn((m, k), generator=gen).to(din)
        b = (torch.randn((n, k) if layout == L.B_NK else (k, n), generator=gen) * 0.1).to(din)
        out = G.gemm_with_kernel(a.to(DEV), b.to(DEV), kernel, dout, layout)
        torch.cuda.synchronize()
        if din == torch.float32:
            ref = (a.double() @ (b.double().T if layout == L.B_NK else b.double()))
            chk = orc.check_result(out.cpu().numpy(), ref.numpy())
            assert chk["correct"], chk
        else:
            _check_tolerance(out.cpu(), a, b, layout, dout)
        ran += 1
    assert ran > 0, "the rung accepts none of the small shapes"


def _random_selection_cases(count=48, seed=2026):
    """Seeded random problems for the default selection: M log-uniform in
    [1, 2048), N in [1, 8192), K in [1, 4096), N and K rounded down to a
    multiple of 8 three times in four (so the 16-byte-row kernels get their
    share), a random dtype pair and layout, at most 2e9 multiply-adds each.
    With this seed the selection spreads them over mfma_staged,
    splitk_decode, fp32_tiled, mfma_direct and gemv_decode."""
    rng = np.random.RandomState(seed)

    def dim(hi):
        v = int(np.exp(rng.uniform(0, np.log(hi))))
        return max(8, v // 8 * 8) if rng.uniform() < 0.75 else v

    cases = []
    while len(cases) < count:
        m = int(np.exp(rng.uniform(0, np.log(2048))))
        n, k = dim(8192), dim(4096)
        if m * n * k > 2e9:
            continue
        din, dout = PAIRS[rng.randint(len(PAIRS))]
        layout = (L.B_NK, L.B_KN)[rng.randint(2)]
        cases.append(pytest.param(m, n, k, layout, din, dout,
                                  id=f"M{m}-N{n}-K{k}-{LAYOUT[layout]}-{NAME[din]}-{NAME[dout]}"))
    return cases


@pytest.mark.parametrize("m,n,k,layout,din,dout", _random_selection_cases())
def test_selected_kernel_random_shapes(m, n, k, layout, din, dout):
    """nanovllm::gemm / gemm_kn (whatever kernel the selection picks) on
    seeded random ragged problems, held to the same bars as every rung:
    narrow outputs by the 2-ulp rule, fp32 by the reference's elementwise
    check (common.cuh:18-31)."""
    gen = torch.Generator().manual_seed(m * 7919 + n * 31 + k)
    a = torch.randn((m, k), generator=gen).to(din)
    b = (torch.randn((n, k) if layout == L.B_NK else (k, n), generator=gen) * 0.1).to(din)
    ad, bd = a.to(DEV), b.to(DEV)
    _say(f"selected {G.selected_kernel(ad, bd, dout, layout)} {NAME[din]}->{NAME[dout]} {LAYOUT[layout]} "
         f"M={m} N={n} K={k}")
    out = (G.gemm if layout == L.B_NK else G.gemm_kn)(ad, bd, dout)
    torch.cuda.synchronize()
    assert out.shape == (m, n) and out.dtype == dout
    if din == torch.float32:
        ref = a.double() @ (b.double().T if layout == L.B_NK else b.double())
        chk = orc.check_result(out.cpu().numpy(), ref.numpy())
        assert chk["correct"], chk
    else:
        _check_tolerance(out.cpu(), a, b, layout, dout)


def _random_stride_cases(count=32, seed=3031):
    """Seeded random problems with padded leading dimensions: the shapes as
    in _random_selection_cases (at most 5e8 multiply-adds), each of lda,
    ldb and ldc padded by 0, 1, 3, 8 or 16 elements."""
    rng = np.random.RandomState(seed)
    pads = (0, 1, 3, 8, 16)
    cases = []
    while len(cases) < count:
        m = int(np.exp(rng.uniform(0, np.log(2048))))
        n, k = (int(np.exp(rng.uniform(0, np.log(hi)))) for hi in (8192, 4096))
        n, k = (max(8, v // 8 * 8) if rng.uniform() < 0.75 else v for v in (n, k))
        if m * n * k > 5e8:
            continue
        din, dout = PAIRS[rng.randint(len(PAIRS))]
        layout = (L.B_NK, L.B_KN)[rng.randint(2)]
        pa, pb, pc = (pads[rng.randint(len(pads))] for _ in range(3))
        cases.append(pytest.param(m, n, k, layout, din, dout, pa, pb, pc,
                                  id=f"M{m}-N{n}-K{k}-{LAYOUT[layout]}-{NAME[din]}-{NAME[dout]}-pad{pa}.{pb}.{pc}"))
    return cases


@pytest.mark.parametrize("m,n,k,layout,din,dout,pa,pb,pc", _random_stride_cases())
def test_selected_kernel_random_padded_strides(m, n, k, layout, din, dout, pa, pb, pc):
    """nanovllm_gemm through the C ABI with lda = K + pa, ldb = (K or N) + pb
    and ldc = N + pc (the selection then sees the leading dimensions' 16-byte
    alignment as well as the shape): the same bars as the contiguous
    problems, and no write into the padding of C."""
    gen = torch.Generator().manual_seed(m * 104729 + n * 131 + k * 7 + pa + 5 * pb + 25 * pc)
    a = torch.randn((m, k), generator=gen).to(din)
    bshape = (n, k) if layout == L.B_NK else (k, n)
    b = (torch.randn(bshape, generator=gen) * 0.1).to(din)
    lda, ldb, ldc = k + pa, bshape[1] + pb, n + pc
    a_full = torch.zeros((m, lda), dtype=din)
    a_full[:, :k] = a
    b_full = torch.zeros((bshape[0], ldb), dtype=din)
    b_full[:, :bshape[1]] = b
    ad, bd = a_full.to(DEV), b_full.to(DEV)
    c = torch.full((m, ldc), 7.0, dtype=dout, device=DEV)
    kid = L.select(m, n, k, lda, ldb, ldc, layout, CODE[din], CODE[dout],
                   ad.data_ptr() % 16 == 0 and bd.data_ptr() % 16 == 0)
    _say(f"selected {L.kernel_name(kid)} {NAME[din]}->{NAME[dout]} {LAYOUT[layout]} M={m} N={n} K={k} "
         f"lda={lda} ldb={ldb} ldc={ldc}")
    L.gemm_raw(ad.data_ptr(), bd.data_ptr(), c.data_ptr(), m, n, k, lda, ldb, ldc, layout, CODE[din], CODE[dout],
               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert bool((c[:, n:] == 7.0).all()), "a padding column of C was written"
    out = c[:, :n].contiguous()
    if din == torch.float32:
        ref = a.double() @ (b.double().T if layout == L.B_NK else b.double())
        chk = orc.check_result(out.cpu().numpy(), ref.numpy())
        assert chk["correct"], chk
    else:
        _check_tolerance(out.cpu(), a, b, layout, dout)


@pytest.mark.parametrize("kernel", [L.KERNEL_FP32_NAIVE, L.KERNEL_FP32_TILED], ids=lambda k: L.kernel_name(k))
@pytest.mark.parametrize("layout", [L.B_KN, L.B_NK], ids=["kn", "nk"])
def test_fp32_reference_known_answer(kernel, layout):
    """The reference's FP32 ladder case (gemm_tiled.cu:228-260, gemm.cu:19-29):
    M, N, K = 127, 193, 65 with a[i] = (i % 19 - 9) * 0.1f and
    b[i] = (i % 13 - 6) * 0.1f in float32, B[K,N] row-major (and the same B
    transposed into W[N,K]), checked as check_result does (common.cuh:18-31:
    |e| <= 1e-4 + 1e-4 |ref| against the double-accumulated product) on both
    FP32 rungs."""
    m, n, k = 127, 193, 65
    a = torch.from_numpy(orc.kat_tiled_a(m, k))
    b_kn = torch.from_numpy(orc.kat_tiled_b(k, n))
    b = b_kn if layout == L.B_KN else b_kn.T.contiguous()
    _say(f"fp32 known answer {L.kernel_name(kernel)} {LAYOUT[layout]}")
    out = G.gemm_with_kernel(a.to(DEV), b.to(DEV), kernel, torch.float32, layout)
    torch.cuda.synchronize()
    ref = orc.gemm_f64(a.double().numpy(), b_kn.double().numpy(), "kn")
    chk = orc.check_result(out.cpu().numpy(), ref.astype(np.float32))
    assert chk["correct"], chk
    assert orc.rel_frobenius(out.cpu().numpy(), ref) <= 1e-5


# The last two take the 64 x 64 tiles (at least 512 of them), the others the
# 64 x 32 tiles.
FP32_BUFFERED_SHAPES = [(1, 4, 4), (3, 8, 60), (64, 64, 64), (65, 68, 68), (130, 196, 132), (127, 192, 260),
                        (200, 256, 1028), (257, 132, 192), (1500, 1400, 68), (1090, 1028, 100)]


@pytest.mark.parametrize("layout", [L.B_KN, L.B_NK], ids=["kn", "nk"])
def test_fp32_buffered_ragged(layout):
    """fp32_tiled on 16-byte rows (K % 4 == 0, N % 4 == 0 for B[K,N]): the
    buffered form, on edge tiles in M and N and K tails that are not a
    multiple of the 32- or 64-wide K-tile, in both tile configurations;
    check_result against the float64 product and relative Frobenius <= 1e-5."""
    gen = torch.Generator().manual_seed(21)
    for m, n, k in FP32_BUFFERED_SHAPES:
        _say(f"fp32 buffered {LAYOUT[layout]} M={m} N={n} K={k}")
        a = torch.rand((m, k), generator=gen) * 2 - 1
        b = torch.rand((n, k) if layout == L.B_NK else (k, n), generator=gen) * 2 - 1
        out = G.gemm_with_kernel(a.to(DEV), b.to(DEV), L.KERNEL_FP32_TILED, torch.float32, layout)
        torch.cuda.synchronize()
        ref = (a.double() @ (b.double().T if layout == L.B_NK else b.double())).numpy()
        got = out.cpu().numpy()
        chk = orc.check_result(got, ref.astype(np.float32))
        assert chk["correct"], (m, n, k, chk)
        assert orc.rel_frobenius(got, ref) <= 1e-5, (m, n, k)


@pytest.mark.parametrize("layout", [L.B_KN, L.B_NK], ids=["kn", "nk"])
@pytest.mark.parametrize("m,n,k", [(130, 196, 132), (1500, 1400, 68)], ids=["tiles64x32", "tiles64x64"])
def test_fp32_buffered_padded_leading_dims(layout, m, n, k):
    """The buffered fp32 form through the C ABI with lda > K and ldb past the
    row length (K + 12 for W[N,K], N + 20 for B[K,N]): the padding holds NaN,
    which must not reach any output; every output element checked."""
    gen = torch.Generator().manual_seed(23 + m)
    lda = k + 8
    rows_b, cols_b = (n, k) if layout == L.B_NK else (k, n)
    ldb = cols_b + (12 if layout == L.B_NK else 20)
    a_full = torch.full((m, lda), float("nan"))
    a_full[:, :k] = torch.rand((m, k), generator=gen) * 2 - 1
    b_full = torch.full((rows_b, ldb), float("nan"))
    b_full[:, :cols_b] = torch.rand((rows_b, cols_b), generator=gen) * 2 - 1
    ad, bd = a_full.to(DEV), b_full.to(DEV)
    c = torch.empty((m, n), device=DEV)
    _say(f"fp32 buffered padded {LAYOUT[layout]} M={m} N={n} K={k} lda={lda} ldb={ldb}")
    L.gemm_raw(ad.data_ptr(), bd.data_ptr(), c.data_ptr(), m, n, k, lda, ldb, n, layout, L.F32, L.F32,
               torch.cuda.current_stream().cuda_stream, L.KERNEL_FP32_TILED)
    torch.cuda.synchronize()
    a64 = a_full[:, :k].double()
    b64 = b_full[:, :cols_b].double()
    ref = (a64 @ (b64.T if layout == L.B_NK else b64)).numpy()
    got = c.cpu().numpy()
    assert np.isfinite(got).all()
    chk = orc.check_result(got, ref.astype(np.float32))
    assert chk["correct"], chk
    assert orc.rel_frobenius(got, ref) <= 1e-5


# ---------------------------------------------------------------------------
# Known-answer inputs: bit-exact on every kernel that takes the shape
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("label,m,n,k", orc.DEFAULT_SHAPES, ids=[s[0] for s in orc.DEFAULT_SHAPES])
@pytest.mark.parametrize("din", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_kat_bit_exact(label, m, n, k, din):
    for layout in (L.B_KN, L.B_NK):
        if layout == L.B_KN:   # gemm_bench.cu generators, B[K,N]
            a_int, b_int = orc.kat_bench_a_int(m, k), orc.kat_bench_b_int(k, n)
        else:                  # gemm_wmma.cu generators, W[N,K]
            a_int, b_int = orc.kat_wmma_a_int(m, k), orc.kat_wmma_w_int(n, k)
        exact = orc.exact_kat_int(a_int, b_int, LAYOUT[layout]).astype(np.float64) / 1024.0
        a = torch.from_numpy(orc.kat_value(a_int)).to(din).to(DEV)
        b = torch.from_numpy(orc.kat_value(b_int)).to(din).to(DEV)
        for dout in (torch.float32, din):
            want = orc.round_f64(exact, NAME[dout])
            ldb = k if layout == L.B_NK else n
            for kernel in KERNELS:
                if not L.kernel_supports(kernel, m, n, k, k, ldb, n, layout, CODE[din], CODE[dout], True):
                    continue
                _say(f"kat {label} {L.kernel_name(kernel)} {NAME[din]}->{NAME[dout]} {LAYOUT[layout]}")
                out = G.gemm_with_kernel(a, b, kernel, dout, layout)
                torch.cuda.synchronize()
                got = _to_np_out(out, dout)
                mism = int((got != want).sum()) if dout != torch.float32 else int((got != want).sum())
                assert mism == 0, f"{mism} elements differ from the exact value"


# ---------------------------------------------------------------------------
# The measured workloads at full size
# ---------------------------------------------------------------------------
WORKLOAD_CASES = [(name, m) for name, wl in W.WORKLOADS.items() for m in wl.ms]


@pytest.mark.parametrize("name,m", WORKLOAD_CASES, ids=[f"{n}-M{m}" for n, m in WORKLOAD_CASES])
def test_workload_parity(name, m):
    wl = W.WORKLOADS[name]
    _say(f"workload {name} M={m} N={wl.n} K={wl.k}")
    a, b = W.make_inputs(name, m)
    ad, bd = a.to(DEV), b.to(DEV)
    if wl.b_layout == L.B_NK:
        out = G.gemm(ad, bd, wl.dtype_out)
    else:
        out = G.gemm_kn(ad, bd, wl.dtype_out)
    torch.cuda.synchronize()
    got = out.cpu()
    if wl.dtype_in == torch.float32:
        ref32 = torch.matmul(a, b)                      # the reference's own check target
        rel = orc.rel_frobenius(got.numpy(), ref32.numpy())
        assert rel <= 1e-5, rel
        ref64 = (a.double() @ b.double()).numpy()
        assert orc.rel_frobenius(got.numpy(), ref64) <= 1e-5
        assert orc.check_result(got.numpy(), ref64.astype(np.float32))["correct"]
        return
    rows = None
    if m * wl.n * wl.k > 2 ** 36:   # the LM head at M = 512: 64 rows spread over M, all N
        rows = np.unique(np.linspace(0, m - 1, 64).astype(int))
    stats = _check_tolerance(got, a, b, wl.b_layout, wl.dtype_out, rows=rows)
    _say(f"  {name} M={m}: {stats}")


STAGED_GRIDS = [(600, 1000, 1000), (600, 1000, 2056), (1100, 2000, 1000), (2100, 2000, 1000), (2100, 4100, 1000),
                (2100, 7000, 1000)]


@pytest.mark.parametrize("m,n,k", STAGED_GRIDS, ids=["40tiles-64x64", "40tiles-64x64-deep", "144tiles-spread",
                                                     "wide136-128x256", "wide289-2deep", "wide476-128x256"])
@pytest.mark.parametrize("din,dout", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)],
                         ids=["bf16", "f16-f32"])
def test_staged_ring_depths_ragged(m, n, k, din, dout):
    """mfma_staged's tile choices: a grid of at most 128 tiles of 128 x 128
    takes 64 x 64 tiles (3-deep ring, spread copies); up to 256 tiles 128 x
    128 with the spread 3-deep ring; above that 128 x 256 tiles (8 waves,
    3-deep ring, copies spread between the MFMAs) unless there are 257-384
    of those, where 128 x 128 with a 2-deep ring takes over; each on ragged
    M and N and a K that is not a multiple of the 64-wide K-tile (the last
    tile is padded with zeros)."""
    _say(f"staged ring M={m} N={n} K={k} {NAME[din]}->{NAME[dout]}")
    gen = torch.Generator().manual_seed(m + n)
    a = torch.randn((m, k), generator=gen).to(din)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(din)
    out = G.gemm_with_kernel(a.to(DEV), w.to(DEV), L.KERNEL_MFMA_STAGED, dout, L.B_NK)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 48).astype(int), np.arange(m - 16, m)]))
    _check_tolerance(out.cpu(), a, w, L.B_NK, dout, rows=rows)


@pytest.mark.parametrize("din", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_staged_tile_choices_same_bits(din):
    """Every tile choice of mfma_staged sums K in the same order, so a row's
    output does not depend on how many rows share the launch: with N = 4104
    and K = 1000, M = 100 / 600 / 1000 / 2100 select 64 x 64 tiles, 128 x 128
    on the spread 3-deep ring, 128 x 256, and 128 x 128 on the 2-deep burst
    ring, and the first 100 rows (fp32 outputs, so any reordering of the K
    sum would show) are bit-identical across all four."""
    n, k, rows = 4104, 1000, 100
    gen = torch.Generator().manual_seed(4104)
    a = torch.randn((2100, k), generator=gen).to(din)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(din)
    a_d, w_d = a.to(DEV), w.to(DEV)
    first = None
    for m in (100, 600, 1000, 2100):
        _say(f"staged tile choice M={m} N={n} K={k} {NAME[din]}->f32")
        out = G.gemm_with_kernel(a_d[:m], w_d, L.KERNEL_MFMA_STAGED, torch.float32, L.B_NK)
        torch.cuda.synchronize()
        head = out[:rows].cpu()
        if first is None:
            first = head
            _check_tolerance(head, a[:rows], w, L.B_NK, torch.float32)
        else:
            assert torch.equal(head, first), f"M={m}: {int((head != first).sum())} of the first {rows} rows' outputs differ"


@pytest.mark.parametrize("layout", [L.B_NK, L.B_KN], ids=["nk", "kn"])
@pytest.mark.parametrize("dout", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_staged_multi_round_same_bits(layout, dout):
    """A 128 x 256 grid of more than one round on the CUs (M = 512, N =
    33000: 4 x 129 = 516 tiles, a ragged last column of tiles): the first
    100 rows equal, bit for bit, the same rows computed at M = 100 (64 x 64
    tiles), every column, and sampled rows meet the tolerance."""
    m, n, k, rows = 512, 33000, 256, 100
    gen = torch.Generator().manual_seed(33000)
    a = torch.randn((m, k), generator=gen).bfloat16()
    b = (torch.randn((n, k) if layout == L.B_NK else (k, n), generator=gen) * 0.1).bfloat16()
    a_d, b_d = a.to(DEV), b.to(DEV)
    _say(f"staged multi-round M={m} N={n} K={k} layout={layout} bf16->{NAME[dout]}")
    full = G.gemm_with_kernel(a_d, b_d, L.KERNEL_MFMA_STAGED, dout, layout)
    small = G.gemm_with_kernel(a_d[:rows], b_d, L.KERNEL_MFMA_STAGED, dout, layout)
    torch.cuda.synchronize()
    head = full[:rows].cpu()
    assert torch.equal(head, small.cpu()), f"{int((head != small.cpu()).sum())} outputs differ"
    sample = torch.arange(0, m, 37)
    _check_tolerance(full.cpu()[sample], a[sample], b, layout, dout)


@pytest.mark.parametrize("din", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_staged_square256_same_bits(din):
    """fp32 logits over a W larger than the Infinity Cache take 256 x 256
    tiles whose C tile leaves LDS in two passes of 128 rows: M = 500, N =
    140001, K = 1000 (W 280 MB; 2 x 547 tiles, a ragged last column, a
    last tile row that ends inside its second pass, a K tail).  Rows 0-99
    and 400-499 equal, bit for bit, the same rows computed alone (M = 100:
    128 x 256 tiles), every column, and rows on both sides of each pass
    boundary meet the tolerance."""
    m, n, k = 500, 140001, 1000
    gen = torch.Generator().manual_seed(140001)
    a = torch.randn((m, k), generator=gen).to(din)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(din)
    a_d, w_d = a.to(DEV), w.to(DEV)
    _say(f"staged 256x256 M={m} N={n} K={k} {NAME[din]}->f32")
    full = G.gemm_with_kernel(a_d, w_d, L.KERNEL_MFMA_STAGED, torch.float32, L.B_NK)
    torch.cuda.synchronize()
    for r0 in (0, 400):
        part = G.gemm_with_kernel(a_d[r0:r0 + 100], w_d, L.KERNEL_MFMA_STAGED, torch.float32, L.B_NK)
        torch.cuda.synchronize()
        head = full[r0:r0 + 100].cpu()
        assert torch.equal(head, part.cpu()), f"rows {r0}-{r0 + 99}: {int((head != part.cpu()).sum())} outputs differ"
    rows = np.array([0, 1, 127, 128, 129, 255, 256, 383, 384, 385, 498, 499])
    _check_tolerance(full.cpu(), a, w, L.B_NK, torch.float32, rows=rows)
    del full, w_d


def test_staged_square256_padded_ldc():
    """The 256 x 256 tiles with a C row stride that is not a multiple of 16
    bytes (ldc = N + 3 fp32): every tile of both 128-row passes takes the
    element-wise store.  Equal, bit for bit, to the same product into a
    dense C, and the 3 padding columns of every row keep their sentinel."""
    m, n, k = 512, 140000, 1024
    gen = torch.Generator().manual_seed(140000)
    a = torch.randn((m, k), generator=gen).bfloat16().to(DEV)
    w = (torch.randn((n, k), generator=gen) * 0.1).bfloat16().to(DEV)
    _say(f"staged 256x256 padded ldc M={m} N={n} K={k}")
    dense = G.gemm_with_kernel(a, w, L.KERNEL_MFMA_STAGED, torch.float32, L.B_NK)
    ldc = n + 3
    padded = torch.full((m, ldc), 7.0, dtype=torch.float32, device=DEV)
    L.gemm_raw(a.data_ptr(), w.data_ptr(), padded.data_ptr(), m, n, k, k, k, ldc, L.B_NK, L.BF16, L.F32,
               torch.cuda.current_stream().cuda_stream, kernel=L.KERNEL_MFMA_STAGED)
    torch.cuda.synchronize()
    assert torch.equal(padded[:, :n], dense), f"{int((padded[:, :n] != dense).sum())} outputs differ"
    assert bool((padded[:, n:] == 7.0).all()), "a padding column was written"
    del a, w, dense, padded


STAGED_GRIDS_KN = [(600, 1000, 1000), (1100, 2000, 1000), (2100, 2000, 1000), (2100, 4104, 1000),
                   (2100, 7000, 1000), (40, 520, 72), (2048, 4096, 1024), (1, 6144, 1024), (5, 200, 136)]


@pytest.mark.parametrize("m,n,k", STAGED_GRIDS_KN, ids=["40tiles-64x64", "144tiles-128x128", "wide136-128x256",
                                                        "wide289-128x128-2deep", "wide476-128x256", "tiny",
                                                        "headline", "decode", "ragged-small"])
@pytest.mark.parametrize("din,dout", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)],
                         ids=["bf16", "f16-f32"])
def test_staged_kn_ragged(m, n, k, din, dout):
    """mfma_staged on B[K,N] (the reference bench's layout, gemm_bench.cu:103-106,
    117-196): every tile choice and copy schedule of the grid-size table, B's
    k-rows copied as they lie and read back with the transposing fragment
    read; ragged M, N a multiple of 8 but not of the tile, K not a multiple
    of the 64-wide K-tile, decode-sized M."""
    _say(f"staged B[K,N] M={m} N={n} K={k} {NAME[din]}->{NAME[dout]}")
    gen = torch.Generator().manual_seed(m + 3 * n)
    a = torch.randn((m, k), generator=gen).to(din)
    b = (torch.randn((k, n), generator=gen) * 0.1).to(din)
    want = L.KERNEL_SPLITK_DECODE if m <= 32 or (m <= 64 and n <= 4096) else L.KERNEL_MFMA_STAGED
    assert L.select(m, n, k, k, n, n, L.B_KN, CODE[din], CODE[dout], True) == want
    out = G.gemm_with_kernel(a.to(DEV), b.to(DEV), L.KERNEL_MFMA_STAGED, dout, L.B_KN)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 48).astype(int), np.arange(max(m - 16, 0), m)]))
    _check_tolerance(out.cpu(), a, b, L.B_KN, dout, rows=rows)
    # The same product from W[N,K] = B^T sums K in the same order: bit-identical.
    out_nk = G.gemm_with_kernel(a.to(DEV), b.t().contiguous().to(DEV), L.KERNEL_MFMA_STAGED, dout, L.B_NK)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out_nk.cpu())


SPLITK_KN_CASES = [(1, 6144, 1024), (5, 200, 136), (8, 8224, 1000), (16, 1024, 2048), (13, 520, 1000),
                   (29, 4104, 520), (33, 1000, 72), (64, 7168, 1024)]


@pytest.mark.parametrize("m,n,k", SPLITK_KN_CASES, ids=[f"M{m}-N{n}-K{k}" for m, n, k in SPLITK_KN_CASES])
@pytest.mark.parametrize("din,dout", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)],
                         ids=["bf16", "f16-f32"])
def test_splitk_kn_ragged(m, n, k, din, dout):
    """splitk_decode on B[K,N] (the reference bench's layout) up to M = 64:
    64 columns per workgroup, B's k-rows copied as they lie and read back
    with the transposing LDS read; N a multiple of 8 but not of 64 (the last
    workgroup's chunks past N read the last chunk and are not stored), K
    ending in a partial 64-row line (zeros past K), every A-row count.  Up to
    M = 8, and with N below 65536 (every case here), both layouts use 16 K
    partitions in the same order, so the product equals the W[N,K]
    splitk_decode result bit for bit."""
    _say(f"splitk B[K,N] M={m} N={n} K={k} {NAME[din]}->{NAME[dout]}")
    gen = torch.Generator().manual_seed(5 * m + n + k)
    a = torch.randn((m, k), generator=gen).to(din)
    b = (torch.randn((k, n), generator=gen) * 0.1).to(din)
    want = L.KERNEL_SPLITK_DECODE if m <= 32 or n <= 4096 else L.KERNEL_MFMA_STAGED
    assert L.select(m, n, k, k, n, n, L.B_KN, CODE[din], CODE[dout], True) == want
    out = G.gemm_with_kernel(a.to(DEV), b.to(DEV), L.KERNEL_SPLITK_DECODE, dout, L.B_KN)
    torch.cuda.synchronize()
    _check_tolerance(out.cpu(), a, b, L.B_KN, dout)
    if m <= 8:
        out_nk = G.gemm_with_kernel(a.to(DEV), b.t().contiguous().to(DEV), L.KERNEL_SPLITK_DECODE, dout, L.B_NK)
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), out_nk.cpu())


@pytest.mark.parametrize("m", [1, 5, 13, 29])
def test_splitk_wide_n_ragged(m):
    """splitk_decode on N >= 65536: M <= 16 32 rows and M <= 32 128 rows per
    workgroup; a ragged N leaves the last workgroup partly past N (clamped
    copies, masked stores)."""
    n, k = 70001, 256
    _say(f"splitk wide N={n} M={m} K={k}")
    gen = torch.Generator().manual_seed(m)
    a = torch.randn((m, k), generator=gen).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(torch.bfloat16)
    out = G.gemm_with_kernel(a.to(DEV), w.to(DEV), L.KERNEL_SPLITK_DECODE, torch.float32, L.B_NK)
    torch.cuda.synchronize()
    _check_tolerance(out.cpu(), a, w, L.B_NK, torch.float32)


SPLITK_CONFIG_CASES = ([(1000, 3592, m) for m in (1, 9, 20, 32)] + [(3000, 1000, m) for m in (1, 7, 16, 25)]
                       + [(8224, 1000, m) for m in (3, 12, 29)] + [(16400, 520, m) for m in (5, 16, 32)])


@pytest.mark.parametrize("n,k,m", SPLITK_CONFIG_CASES, ids=[f"N{n}-K{k}-M{m}" for n, k, m in SPLITK_CONFIG_CASES])
@pytest.mark.parametrize("din,dout", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)],
                         ids=["bf16", "f16-f32"])
def test_splitk_configs_ragged(n, k, m, din, dout):
    """The LDS-staged splitk_decode configurations below the LM head: at most
    2048 W rows (16 rows per workgroup, 16 or 8 waves) and above (32 rows
    while 32-row workgroups fit the CUs; 48 rows, or 8-wave workgroups
    several to a CU, on wider N: 8224 and 16400 rows), every A-row count
    (8, 16, 32), a ragged N and a K that ends in a partial 64-element line
    (3592 = 56 x 64 + 8, 1000 = 15 x 64 + 40, 520 = 8 x 64 + 8), so the last
    line copies zeros past K into both W and A."""
    _say(f"splitk config N={n} K={k} M={m} {NAME[din]}->{NAME[dout]}")
    gen = torch.Generator().manual_seed(n + k + m)
    a = torch.randn((m, k), generator=gen).to(din)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(din)
    out = G.gemm_with_kernel(a.to(DEV), w.to(DEV), L.KERNEL_SPLITK_DECODE, dout, L.B_NK)
    torch.cuda.synchronize()
    _check_tolerance(out.cpu(), a, w, L.B_NK, dout)


# (N, A-row counts that share one K-partition order).  Below 65536 W rows
# every M from 2 to 32 uses 16 partitions; the LM-head width uses 8
# partitions for M = 1-16 and 4 for M = 17-32.
SPLITK_SAME_ORDER = [(6144, (2, 8, 13, 16, 32)), (1000, (2, 8, 13, 16, 32)), (151936, (1, 2, 8, 13, 16)),
                     (151936, (17, 24, 32))]


@pytest.mark.parametrize("n,ms", SPLITK_SAME_ORDER, ids=["N6144", "N1000", "N151936-M1to16", "N151936-M17to32"])
def test_splitk_rows_same_bits_across_m(n, ms):
    """A row's output from splitk_decode depends only on the number of K
    partitions, which the configurations fix per family (the partition of
    64-element line L is L % PARTS, lines are added in increasing order
    within a partition and partitions in order, whatever the waves, lines
    per wave or W rows per workgroup): the first two rows (fp32 outputs; the
    one row at M = 1) are bit-identical across each listed set of A-row
    counts, on the decode
    width, on a narrow W (16-row workgroups) and on the LM-head width in its
    two partition families."""
    k = 1024
    gen = torch.Generator().manual_seed(n + ms[0])
    a = torch.randn((32, k), generator=gen).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(torch.bfloat16)
    a_d, w_d = a.to(DEV), w.to(DEV)
    heads = {}
    for m in ms:
        _say(f"splitk rows across M: M={m} N={n} K={k} bf16->f32")
        out = G.gemm_with_kernel(a_d[:m], w_d, L.KERNEL_SPLITK_DECODE, torch.float32, L.B_NK)
        torch.cuda.synchronize()
        heads[m] = out[:2].cpu()
    first = heads[max(ms)]
    _check_tolerance(first, a[:2], w, L.B_NK, torch.float32)
    for m, head in heads.items():
        rows = head.shape[0]
        assert torch.equal(head, first[:rows]), f"M={m}: {int((head != first[:rows]).sum())} of the first rows' outputs differ"


@pytest.mark.parametrize("n", [6144, 1000], ids=["N6144", "N1000"])
def test_splitk_kn_rows_same_bits_across_m(n):
    """splitk_decode on B[K,N] uses 16 K partitions up to M = 8 and 8 above:
    the first two rows are bit-identical at M = 2, 5, 8 and again at M = 9,
    16, 32."""
    k = 1024
    gen = torch.Generator().manual_seed(3 * n)
    a = torch.randn((32, k), generator=gen).to(torch.bfloat16)
    b = (torch.randn((k, n + 8 - n % 8), generator=gen) * 0.1).to(torch.bfloat16)
    a_d, b_d = a.to(DEV), b.to(DEV)
    for ms in ((2, 5, 8), (9, 16, 32)):
        first = None
        for m in ms:
            _say(f"splitk B[K,N] rows across M: M={m} N={b.shape[1]} K={k}")
            out = G.gemm_with_kernel(a_d[:m], b_d, L.KERNEL_SPLITK_DECODE, torch.float32, L.B_KN)
            torch.cuda.synchronize()
            head = out[:2].cpu()
            if first is None:
                first = head
                _check_tolerance(head, a[:2], b, L.B_KN, torch.float32)
            else:
                assert torch.equal(head, first), f"M={m}: {int((head != first).sum())} outputs differ"


SPLITK64_CASES = [(1000, 3592, 64), (4096, 1000, 33), (5000, 1000, 47), (9000, 1000, 64), (20000, 264, 40)]


@pytest.mark.parametrize("n,k,m", SPLITK64_CASES, ids=[f"N{n}-K{k}-M{m}" for n, k, m in SPLITK64_CASES])
@pytest.mark.parametrize("din,dout", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)],
                         ids=["bf16", "f16-f32"])
def test_splitk_m64_configs_ragged(n, k, m, din, dout):
    """The plain GEMM's 33 <= M <= 64 configurations of splitk_decode (64 A
    rows per line; 16 / 32 / 48 W rows per workgroup up to 4096 / 8192 /
    65535 rows), with a ragged N, M not a multiple of 16 (rows past M repeat
    row M - 1 and are not stored) and K ending in a partial line."""
    _say(f"splitk M<=64 N={n} K={k} M={m} {NAME[din]}->{NAME[dout]}")
    gen = torch.Generator().manual_seed(7 * n + k + m)
    a = torch.randn((m, k), generator=gen).to(din)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(din)
    out = G.gemm_with_kernel(a.to(DEV), w.to(DEV), L.KERNEL_SPLITK_DECODE, dout, L.B_NK)
    torch.cuda.synchronize()
    _check_tolerance(out.cpu(), a, w, L.B_NK, dout)


# ---------------------------------------------------------------------------
# Edge cases and API behaviour
# ---------------------------------------------------------------------------
def test_empty_and_degenerate():
    a = torch.randn(0, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(32, 64, device=DEV, dtype=torch.bfloat16)
    assert G.gemm(a, w).shape == (0, 32)
    a = torch.randn(3, 1, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(5, 1, device=DEV, dtype=torch.bfloat16)
    out = G.gemm(a, w, torch.float32)
    assert torch.equal(out.cpu(), (a.float() * w.float().T).cpu())  # K = 1: single exact product


def test_leading_dims_flatten():
    gen = torch.Generator().manual_seed(5)
    a = torch.randn(2, 3, 40, 128, generator=gen).bfloat16()
    w = (torch.randn(96, 128, generator=gen) * 0.1).bfloat16()
    out = G.gemm(a.to(DEV), w.to(DEV))
    assert out.shape == (2, 3, 40, 96)
    flat = G.gemm(a.reshape(-1, 128).to(DEV), w.to(DEV))
    assert torch.equal(out.reshape(-1, 96), flat)


def test_unaligned_pointer_takes_direct_and_is_correct():
    gen = torch.Generator().manual_seed(6)
    m, n, k = 48, 80, 128
    store = torch.randn(m * k + 1, generator=gen).bfloat16().to(DEV)
    a = store[1:].view(m, k)                       # 2-byte offset: not 16-byte aligned
    w = (torch.randn(n, k, generator=gen) * 0.1).bfloat16().to(DEV)
    assert a.data_ptr() % 16 != 0
    assert G.selected_kernel(a, w) == "mfma_direct"
    out = G.gemm(a, w)
    _check_tolerance(out.cpu(), a.cpu(), w.cpu(), L.B_NK, torch.bfloat16)


@pytest.mark.parametrize("kernel", [L.KERNEL_FP32_TILED, L.KERNEL_MFMA_DIRECT, L.KERNEL_MFMA_STAGED,
                                    L.KERNEL_SPLITK_DECODE, L.KERNEL_GEMV_DECODE], ids=lambda k: L.kernel_name(k))
def test_guard_bands_untouched(kernel):
    """Write through the C ABI into a padded C (ldc > n, a row of canaries
    above and below): nothing outside the M x N window may change."""
    din = torch.float32 if kernel == L.KERNEL_FP32_TILED else torch.bfloat16
    dout = torch.float32 if kernel == L.KERNEL_FP32_TILED else torch.bfloat16
    m = {L.KERNEL_SPLITK_DECODE: 20, L.KERNEL_GEMV_DECODE: 1}.get(kernel, 150)
    n, k, pad = 301, 200, 7
    ldc = n + pad
    gen = torch.Generator().manual_seed(8)
    a = torch.randn(m, k, generator=gen).to(din).to(DEV)
    w = (torch.randn(n, k, generator=gen) * 0.1).to(din).to(DEV)
    canary = -12345.0
    buf = torch.full(((m + 2) * ldc,), canary, dtype=dout, device=DEV)
    c_ptr = buf.data_ptr() + ldc * buf.element_size()
    _say(f"guard {L.kernel_name(kernel)} M={m} N={n} K={k} ldc={ldc}")
    L.gemm_raw(a.data_ptr(), w.data_ptr(), c_ptr, m, n, k, k, k, ldc, L.B_NK, CODE[din], CODE[dout],
               torch.cuda.current_stream().cuda_stream, kernel)
    torch.cuda.synchronize()
    full = buf.view(m + 2, ldc).cpu()
    assert (full[0] == canary).all() and (full[-1] == canary).all()
    assert (full[1:-1, n:] == canary).all()
    ref = G.gemm_with_kernel(a, w, L.KERNEL_MFMA_DIRECT if din != torch.float32 else L.KERNEL_FP32_NAIVE, dout)
    if din == torch.float32:
        assert orc.check_result(full[1:-1, :n].numpy(), ref.cpu().numpy())["correct"]
    else:
        _check_tolerance(full[1:-1, :n], a.cpu(), w.cpu(), L.B_NK, dout)


def test_runs_on_current_stream():
    gen = torch.Generator().manual_seed(9)
    a = torch.randn(64, 256, generator=gen).bfloat16().to(DEV)
    w = (torch.randn(512, 256, generator=gen) * 0.1).bfloat16().to(DEV)
    ref = G.gemm(a, w)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        out = G.gemm(a, w)
    side.synchronize()
    assert torch.equal(out, ref)


def test_deterministic():
    a, w = W.make_inputs("bf16_prefill_2048x4096x1024", 2048, device=DEV)
    x = G.gemm(a, w)
    y = G.gemm(a, w)
    a2, w2 = W.make_inputs("bf16_decode_n6144_k1024", 16, device=DEV)
    assert torch.equal(x, y)
    assert torch.equal(G.gemm(a2, w2), G.gemm(a2, w2))


@pytest.mark.parametrize("m", [8, 256])
def test_graph_capture_replay(m):
    """Capture the op in a HIP graph, replay it with new inputs several times
    with eager work in between, and compare every replay with eager
    (pattern of tests/kernels/test_fused_add_rmsnorm.py:127-147)."""
    gen = torch.Generator().manual_seed(10)
    k, n = 512, 1024
    a_static = torch.zeros(m, k, dtype=torch.bfloat16, device=DEV)
    w = (torch.randn(n, k, generator=gen) * 0.05).bfloat16().to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        G.gemm(a_static, w)        # warm up outside capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = G.gemm(a_static, w)
    for step in range(4):
        new_a = torch.randn(m, k, generator=gen).bfloat16().to(DEV)
        a_static.copy_(new_a)
        graph.replay()
        eager = G.gemm(new_a, w)
        torch.cuda.synchronize()
        assert torch.equal(out_static, eager), f"replay {step} differs"


def test_graph_capture_first_call_wide_w():
    """A wide-W splitk_decode configuration whose first call is inside graph
    capture (bf16 -> fp32, M = 12, 12000 rows: the configuration is chosen
    with the runtime's occupancy query, which enqueues nothing): the
    captured launch equals eager on every replay."""
    gen = torch.Generator().manual_seed(12)
    m, n, k = 12, 12000, 512
    a_static = torch.randn(m, k, generator=gen).bfloat16().to(DEV)
    w = (torch.randn(n, k, generator=gen) * 0.05).bfloat16().to(DEV)
    _say(f"graph capture, first call M={m} N={n} K={k} bf16->f32")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            out_static = G.gemm(a_static, w, torch.float32)
    torch.cuda.current_stream().wait_stream(side)
    for step in range(3):
        new_a = torch.randn(m, k, generator=gen).bfloat16().to(DEV)
        a_static.copy_(new_a)
        graph.replay()
        eager = G.gemm(new_a, w, torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(out_static, eager), f"replay {step} differs"


def test_torch_compile_fullgraph():
    gen = torch.Generator().manual_seed(12)
    a = torch.randn(40, 256, generator=gen).bfloat16().to(DEV)
    w = (torch.randn(384, 256, generator=gen) * 0.1).bfloat16().to(DEV)

    def f(x, y):
        return torch.ops.nanovllm.gemm(x, y, torch.float32) * 2.0

    compiled = torch.compile(f, fullgraph=True)
    assert torch.equal(compiled(a, w), f(a, w))


def test_cpp_registration_matches_ctypes_path():
    """The C++ registration of nanovllm::gemm / gemm_kn (the default when
    built) gives the ctypes path's bits on every dtype pair and both
    layouts, and raises the Python contract's message for each violation."""
    assert G.REGISTRATION == "torch_library"
    gen = torch.Generator().manual_seed(41)
    for din, dout in ((torch.float32, None), (torch.float16, None), (torch.float16, torch.float32),
                      (torch.bfloat16, None), (torch.bfloat16, torch.float32)):
        for m in (1, 7, 300):
            a = torch.randn(2, m, 96, generator=gen).to(din).to(DEV)
            w = (torch.randn(136, 96, generator=gen) * 0.1).to(din).to(DEV)
            b = (torch.randn(96, 136, generator=gen) * 0.1).to(din).to(DEV)
            assert torch.equal(torch.ops.nanovllm.gemm(a, w, dout), G._launch(a, w, dout, L.B_NK))
            assert torch.equal(torch.ops.nanovllm.gemm_kn(a, b, dout), G._launch(a, b, dout, L.B_KN))
    a = torch.randn(4, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(8, 64, device=DEV, dtype=torch.bfloat16)
    bad = [
        (a, w.half(), None),
        (a, torch.randn(64, 8, device=DEV, dtype=torch.bfloat16).T, None),
        (a, torch.randn(8, 32, device=DEV, dtype=torch.bfloat16), None),
        (a, w, torch.float16),
        (a.int(), w.int(), None),
        (a, w.reshape(2, 4, 64), None),
        (a.T, torch.randn(8, 4, device=DEV, dtype=torch.bfloat16), None),
        (torch.empty(4, 0, device=DEV, dtype=torch.bfloat16), torch.empty(8, 0, device=DEV, dtype=torch.bfloat16),
         None),
    ]
    for x, y, od in bad:
        reason = G.contract_reason(x, y, od)
        assert reason is not None
        with pytest.raises(RuntimeError) as err:
            torch.ops.nanovllm.gemm(x, y, od)
        assert str(err.value).splitlines()[0] == f"nanovllm::gemm: {reason}"
    kn_reason = G.contract_reason(a, torch.randn(32, 8, device=DEV, dtype=torch.bfloat16), None, L.B_KN)
    with pytest.raises(RuntimeError) as err:
        torch.ops.nanovllm.gemm_kn(a, torch.randn(32, 8, device=DEV, dtype=torch.bfloat16))
    assert str(err.value).splitlines()[0] == f"nanovllm::gemm: {kn_reason}"


def test_contract_errors_on_gpu():
    a = torch.randn(4, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(8, 64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="same dtype"):
        G.gemm(a, w.half())
    with pytest.raises(RuntimeError, match="w must be contiguous"):
        G.gemm(a, torch.randn(64, 8, device=DEV, dtype=torch.bfloat16).T)
    with pytest.raises(RuntimeError, match=r"a.size\(-1\)"):
        G.gemm(a, torch.randn(8, 32, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="out_dtype"):
        G.gemm(a, w, torch.float16)


def test_linear_backends_on_gpu():
    gen = torch.Generator().manual_seed(13)
    x = torch.randn(24, 256, generator=gen).bfloat16().to(DEV)
    w = (torch.randn(640, 256, generator=gen) * 0.1).bfloat16().to(DEV)
    bias = torch.randn(640, generator=gen).bfloat16().to(DEV)
    y_hip = G.linear(x, w, bias, backend="hip")
    assert torch.equal(y_hip, G.gemm(x, w) + bias)
    assert torch.equal(G.linear(x, w, bias, backend="auto"), y_hip)
    y_torch = G.linear(x, w, bias, backend="torch").float()
    assert torch.allclose(y_hip.float(), y_torch, atol=0.05, rtol=0.02)


# ---------------------------------------------------------------------------
# Output rounding: round to nearest, ties to even, on every kernel
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("din", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_output_rounding_ties_to_even(din):
    """C[m, n] = a_m * w_n exactly (one non-zero K term), with a = +-(1 + i/s)
    and w = 1 + j/s exact in the input type: many products fall exactly half
    way between two output values, so truncation, ties-away or double
    rounding would differ from the oracle's single RNE in some element."""
    step = 128.0 if din == torch.bfloat16 else 1024.0
    m, n, k = 64, 96, 8
    a = torch.zeros(m, k, dtype=torch.float64)
    w = torch.zeros(n, k, dtype=torch.float64)
    idx_m = torch.arange(m, dtype=torch.float64)
    idx_n = torch.arange(n, dtype=torch.float64)
    a[:, 0] = (1.0 + torch.remainder(idx_m * 3, step) / step) * torch.where(torch.arange(m) % 2 == 0, 1.0, -1.0)
    w[:, 0] = 1.0 + torch.remainder(idx_n * 5, step) / step
    a_t, w_t = a.to(din), w.to(din)
    assert torch.equal(a_t.double(), a) and torch.equal(w_t.double(), w)   # inputs exact
    exact = (a @ w.T).numpy()
    want = orc.round_f64(exact, NAME[din])
    ad, wd = a_t.to(DEV), w_t.to(DEV)
    ran = 0
    for kernel in KERNELS:
        for mm in (1, 32, m):
            if not L.kernel_supports(kernel, mm, n, k, k, k, n, L.B_NK, CODE[din], CODE[din], True):
                continue
            _say(f"rounding {L.kernel_name(kernel)} {NAME[din]} M={mm}")
            out = G.gemm_with_kernel(ad[:mm].contiguous(), wd, kernel, din)
            torch.cuda.synchronize()
            got = _to_np_out(out, din)
            assert np.array_equal(got, want[:mm]), f"{L.kernel_name(kernel)}: {int((got != want[:mm]).sum())} differ"
            ran += 1
    assert ran >= 6   # direct x3, staged x3, splitk x2, gemv x1


# ---------------------------------------------------------------------------
# Fused gate/up projection + SiLU-and-mul
# ---------------------------------------------------------------------------
def _check_silu_mul(got: torch.Tensor, a: torch.Tensor, w: torch.Tensor, dout: torch.dtype, rows=None):
    """Bar: |out - R| <= silu_mul_tolerance (2 ulp of the output type at the
    exact value R = silu(g) u, plus the propagated fp32 accumulation error of
    g and u, plus the fp32 evaluation of silu and the product); for narrow
    outputs also every element within 2 ulp of the fp32 reference
    silu(g32) u32 (fp32 sums on the host, SiLU and product in fp32, rounded
    once) but a few cancellation elements (oracle.narrow_parity);
    for fp32 outputs relative Frobenius <= 1e-5."""
    a64, w64 = a.double().numpy(), w.double().numpy()
    a_rows = a if rows is None else a[rows]
    if rows is not None:
        a64, got = a64[rows], got[rows]
    n = w64.shape[0] // 2
    r, g, u = orc.silu_mul_f64(a64, w64)
    sg, su = orc.abs_products_f64(a64, w64[:n]), orc.abs_products_f64(a64, w64[n:])
    tol = orc.silu_mul_tolerance(r, g, u, sg, su, a.shape[1], NAME[dout])
    g64 = got.double().cpu().numpy()
    assert np.isfinite(g64).all(), "non-finite output"
    err = np.abs(g64 - r)
    bad = err > tol
    assert not bad.any(), f"{int(bad.sum())} elements outside tolerance; worst excess {float((err - tol).max()):.3g}"
    if dout == torch.float32:
        assert orc.rel_frobenius(g64, r) <= 1e-5
    else:
        g32 = a_rows.float() @ w[:n].float().T
        u32 = a_rows.float() @ w[n:].float().T
        ref = _to_np_out((torch.nn.functional.silu(g32) * u32).to(dout), dout)
        # magnitude of the terms of silu(g) u: each sum's terms, weighted by
        # the other factor and the SiLU slope bound
        scale = orc.SILU_SLOPE_BOUND * sg * np.abs(u) + np.abs(orc.silu_f64(g)) * su
        _assert_narrow(orc.narrow_parity(_to_np_out(got, dout), ref, r, scale, NAME[dout]), NAME[dout])


SILU_SHAPES = [(1, 1, 8), (1, 37, 64), (5, 7, 72), (16, 100, 136), (31, 65, 264), (33, 129, 520),
               (130, 300, 264), (257, 97, 1000)]
SILU_KERNELS = [L.KERNEL_GEMV_DECODE, L.KERNEL_SPLITK_DECODE, L.KERNEL_MFMA_STAGED]
SILU_PAIRS = [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32), (torch.float16, torch.float16),
              (torch.float16, torch.float32)]


@pytest.mark.parametrize("kernel", SILU_KERNELS, ids=lambda k: L.kernel_name(k))
@pytest.mark.parametrize("din,dout", SILU_PAIRS, ids=lambda d: NAME[d])
def test_silu_mul_every_rung_small(kernel, din, dout):
    gen = torch.Generator().manual_seed(31)
    ran = 0
    for m, n, k in SILU_SHAPES:
        if kernel == L.KERNEL_GEMV_DECODE and m != 1 or kernel == L.KERNEL_SPLITK_DECODE and m > 64:
            continue
        _say(f"silu_mul {L.kernel_name(kernel)} {NAME[din]}->{NAME[dout]} M={m} N={n} K={k}")
        a = torch.randn((m, k), generator=gen).to(din)
        w = (torch.randn((2 * n, k), generator=gen) * 0.1).to(din)
        out = G.gemm_silu_mul_with_kernel(a.to(DEV), w.to(DEV), kernel, dout)
        torch.cuda.synchronize()
        assert out.shape == (m, n) and out.dtype == dout
        _check_silu_mul(out.cpu(), a, w, dout)
        ran += 1
    assert ran > 0


def _silu_random_cases(count=16, seed=4047):
    """Seeded random problems for the fused op's default selection: M
    log-uniform in [1, 2048), N (output columns, W has 2N rows) in [1, 4096),
    K a multiple of 8 in [8, 4096), a random half-precision input and output
    type, at most 1e9 multiply-adds."""
    rng = np.random.RandomState(seed)
    cases = []
    while len(cases) < count:
        m = int(np.exp(rng.uniform(0, np.log(2048))))
        n = int(np.exp(rng.uniform(0, np.log(4096))))
        k = max(8, int(np.exp(rng.uniform(np.log(8), np.log(4096)))) // 8 * 8)
        if m * 2 * n * k > 1e9:
            continue
        din, dout = SILU_PAIRS[rng.randint(len(SILU_PAIRS))]
        cases.append(pytest.param(m, n, k, din, dout, id=f"M{m}-N{n}-K{k}-{NAME[din]}-{NAME[dout]}"))
    return cases


@pytest.mark.parametrize("m,n,k,din,dout", _silu_random_cases())
def test_silu_mul_selected_random_shapes(m, n, k, din, dout):
    """nanovllm::gemm_silu_mul (the kernel its selection picks) on seeded
    random problems, held to the fused op's bar."""
    gen = torch.Generator().manual_seed(m * 7919 + n * 31 + k)
    a = torch.randn((m, k), generator=gen).to(din)
    w = (torch.randn((2 * n, k), generator=gen) * 0.1).to(din)
    ad, wd = a.to(DEV), w.to(DEV)
    _say(f"silu_mul selected {G.silu_mul_selected_kernel(ad, wd, dout)} {NAME[din]}->{NAME[dout]} M={m} N={n} K={k}")
    out = G.gemm_silu_mul(ad, wd, dout)
    torch.cuda.synchronize()
    assert out.shape == (m, n) and out.dtype == dout
    _check_silu_mul(out.cpu(), a, w, dout)


@pytest.mark.parametrize("m", [1, 4, 32, 48, 2048])
def test_silu_mul_qwen_mlp_shape(m):
    """Qwen3.5-0.8B gate_up_proj (2 x 3584 rows, K = 1024) + SiluAndMul on
    the kernel the selection table picks."""
    gen = torch.Generator().manual_seed(50 + m)
    a = torch.randn((m, 1024), generator=gen).bfloat16()
    w = (torch.randn((7168, 1024), generator=gen) * 0.02).bfloat16()
    ad, wd = a.to(DEV), w.to(DEV)
    want = {1: "splitk_decode", 4: "splitk_decode", 32: "splitk_decode", 48: "splitk_decode",
            2048: "mfma_staged"}[m]
    assert G.silu_mul_selected_kernel(ad, wd) == want
    _say(f"silu_mul qwen mlp M={m} ({want})")
    out = G.gemm_silu_mul(ad, wd)
    torch.cuda.synchronize()
    rows = None if m <= 32 else np.unique(np.concatenate([np.linspace(0, m - 1, 48).astype(int), [m - 1]]))
    _check_silu_mul(out.cpu(), a, w, torch.bfloat16, rows=rows)


@pytest.mark.parametrize("m", [3, 20])
def test_silu_mul_splitk_wide(m):
    """Fused SiLU-and-mul on splitk_decode with 2 N >= 65536 W rows (the wide
    configurations, gate/up group pairs in 32- and 128-row workgroups),
    ragged N and K."""
    n, k = 33001, 136
    _say(f"silu_mul splitk wide M={m} N={n} K={k}")
    gen = torch.Generator().manual_seed(90 + m)
    a = torch.randn((m, k), generator=gen).bfloat16()
    w = (torch.randn((2 * n, k), generator=gen) * 0.1).bfloat16()
    out = G.gemm_silu_mul_with_kernel(a.to(DEV), w.to(DEV), L.KERNEL_SPLITK_DECODE, torch.bfloat16)
    torch.cuda.synchronize()
    _check_silu_mul(out.cpu(), a, w, torch.bfloat16)


def test_silu_mul_contract_errors_on_gpu():
    a = torch.randn(4, 64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="equal height"):
        G.gemm_silu_mul(a, torch.randn(7, 64, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        G.gemm_silu_mul(a.float(), torch.randn(8, 64, device=DEV))
    # a contiguous view two bytes into its storage: rows are not 16-byte aligned
    misaligned = torch.randn(4 * 64 + 1, device=DEV, dtype=torch.bfloat16)[1:].view(4, 64)
    assert misaligned.is_contiguous() and misaligned.data_ptr() % 16 == 2
    with pytest.raises(RuntimeError, match="aligned"):
        G.gemm_silu_mul(misaligned, torch.randn(8, 64, device=DEV, dtype=torch.bfloat16))


# ---------------------------------------------------------------------------
# Greedy LM head (argmax without logits)
# ---------------------------------------------------------------------------
ARGMAX_CASES = [(L.KERNEL_SPLITK_DECODE, m) for m in (1, 5, 17, 32)] + [(L.KERNEL_MFMA_STAGED, m) for m in (1, 33, 300)]


@pytest.mark.parametrize("kernel,m", ARGMAX_CASES, ids=[f"{L.kernel_name(k)}-M{m}" for k, m in ARGMAX_CASES])
@pytest.mark.parametrize("n", [1000, 9000, 70001])
@pytest.mark.parametrize("din", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("rank", ["model", "f32"])
def test_argmax_equals_argmax_of_own_logits(kernel, m, n, din, rank):
    """The greedy head and the fp32-output GEMM on the same kernel compute the
    same fp32 logits.  Ranking the model dtype (the default, the
    reference's), the tokens are exactly torch.argmax of those logits rounded
    to the input type -- which is also the narrow-output GEMM on the same
    kernel -- and the values the chosen rounded logits; ranking fp32, the
    argmax of the fp32 logits.  Rows 3 and n - 2 of W are copies of row 1,
    so some logits tie exactly (first index wins).  The tokens are also
    admissible against the float64 logits."""
    gen = torch.Generator().manual_seed(m * 7 + n)
    k = 256
    a = torch.randn((m, k), generator=gen).to(din)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(din)
    w[3] = w[1]
    w[n - 2] = w[1]
    a[0] = w[1] * 4        # row 0's best token is 1, tied with 3 and n - 2
    ad, wd = a.to(DEV), w.to(DEV)
    _say(f"argmax {L.kernel_name(kernel)} {NAME[din]} M={m} N={n} rank={rank}")
    ldt = None if rank == "model" else torch.float32
    tokens, values = G.gemm_argmax_with_kernel(ad, wd, kernel, ldt)
    logits = G.gemm_with_kernel(ad, wd, kernel, torch.float32)
    narrow = G.gemm_with_kernel(ad, wd, kernel, din) if rank == "model" else None
    torch.cuda.synchronize()
    assert tokens.dtype == torch.int64 and values.dtype == torch.float32
    ranked = logits.to(din).float() if rank == "model" else logits
    if narrow is not None:
        assert torch.equal(narrow.float(), ranked)
    assert torch.equal(tokens, ranked.argmax(-1))
    assert torch.equal(values, ranked.gather(-1, tokens[:, None]).squeeze(-1))
    assert int(tokens[0]) == 1
    a64, w64 = a.double().numpy(), w.double().numpy()
    r = orc.gemm_f64(a64, w64)
    s = orc.abs_products_f64(a64, w64)
    if rank == "model":
        cand = orc.rounded_greedy_candidates(r, s, k, NAME[din])
        assert cand[np.arange(m), tokens.cpu().numpy()].all()
    else:
        assert orc.greedy_token_admissible(tokens.cpu().numpy(), r, s, k).all()


def _argmax_random_cases(count=12, seed=5051):
    """Seeded random problems for the greedy head's default selection: M
    log-uniform in [1, 512), N (vocabulary) in [2, 200000), K a multiple of 8
    in [8, 2048), bf16 or fp16, at most 1e9 multiply-adds and 2e7 logits."""
    rng = np.random.RandomState(seed)
    cases = []
    while len(cases) < count:
        m = int(np.exp(rng.uniform(0, np.log(512))))
        n = int(np.exp(rng.uniform(np.log(2), np.log(200000))))
        k = max(8, int(np.exp(rng.uniform(np.log(8), np.log(2048)))) // 8 * 8)
        if m * n * k > 1e9 or m * n > 2e7:
            continue
        din = (torch.bfloat16, torch.float16)[rng.randint(2)]
        cases.append(pytest.param(m, n, k, din, id=f"M{m}-N{n}-K{k}-{NAME[din]}"))
    return cases


@pytest.mark.parametrize("m,n,k,din", _argmax_random_cases())
def test_argmax_selected_random_shapes(m, n, k, din):
    """nanovllm::gemm_argmax with its default selection on seeded random
    problems: every token is one the reference's greedy rule (argmax of the
    logits rounded to the input type, first index on ties) can return for
    some fp32 summation order of the float64 logits, and its value lies
    within the accumulation bound of that token's float64 logit."""
    gen = torch.Generator().manual_seed(m * 104729 + n * 7 + k)
    a = torch.randn((m, k), generator=gen).to(din)
    w = (torch.randn((n, k), generator=gen) * 0.1).to(din)
    _say(f"argmax selected {NAME[din]} M={m} N={n} K={k}")
    tokens, values = G.gemm_argmax(a.to(DEV), w.to(DEV))
    torch.cuda.synchronize()
    assert tokens.shape == (m,) and tokens.dtype == torch.int64 and values.dtype == torch.float32
    t = tokens.cpu().numpy()
    assert ((t >= 0) & (t < n)).all()
    a64, w64 = a.double().numpy(), w.double().numpy()
    r = orc.gemm_f64(a64, w64)
    s = orc.abs_products_f64(a64, w64)
    cand = orc.rounded_greedy_candidates(r, s, k, NAME[din])
    assert cand[np.arange(m), t].all()
    rows = np.arange(m)
    tol = orc.gemm_tolerance(r[rows, t], s[rows, t], k, NAME[din])
    assert (np.abs(values.cpu().double().numpy() - r[rows, t]) <= tol).all()


@pytest.mark.parametrize("m", [1, 32])
def test_argmax_lm_head_shape_and_graph(m):
    """Qwen3.5 LM head (151936 x 1024): the selected path ranks the bf16
    logits the plain GEMM writes with bf16 output (same configuration), then
    captured in a HIP graph (workspace from the graph's pool) and replayed."""
    gen = torch.Generator().manual_seed(70 + m)
    a = torch.randn((m, 1024), generator=gen).bfloat16().to(DEV)
    w = (torch.randn((151936, 1024), generator=gen) * 0.02).bfloat16().to(DEV)
    _say(f"argmax lm head M={m}")
    tokens, values = G.gemm_argmax(a, w)
    logits = G.gemm(a, w).float()      # bf16 logits from the same splitk configuration
    torch.cuda.synchronize()
    assert torch.equal(tokens, logits.argmax(-1))
    assert torch.equal(values, logits.gather(-1, tokens[:, None]).squeeze(-1))
    a_static = a.clone()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        G.gemm_argmax(a_static, w)
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        t_static, v_static = G.gemm_argmax(a_static, w)
    for step in range(3):
        x = torch.randn((m, 1024), generator=gen).bfloat16().to(DEV)
        a_static.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        t_eager, v_eager = G.gemm_argmax(x, w)
        torch.cuda.synchronize()
        assert torch.equal(t_static, t_eager) and torch.equal(v_static, v_eager), f"replay {step}"


def _exact_head_inputs(m, n, k, seed):
    """Integer numerators over 32 in the ranges of the reference's
    known-answer generators (|a| <= 15/32, |w| <= 14/32): every product is
    a multiple of 1/1024 and every partial sum of K = 1024 of them stays
    below 2^24 / 1024, so the fp32 logits are exact in any summation order.
    Per row of A, an earlier column is planted whose exact logit is just
    below the row's best but rounds to the same bf16 value (the reference's
    first-index rule must pick it; fp32 ranking would not), and the best row
    of W is copied to a later column (an exact tie)."""
    rng = np.random.default_rng(seed)
    a_int = rng.integers(-15, 16, size=(m, k)).astype(np.int64)
    w_int = rng.integers(-14, 15, size=(n, k)).astype(np.int64)
    w64 = w_int.astype(np.float64)      # integer sums below 2^53 are exact in float64
    for i in range(m):
        exact = w64 @ a_int[i].astype(np.float64)
        best = int(exact.argmax())
        w_int[(best + 5000) % n] = w_int[best]                 # exact tie, later column when it wraps
        w64[(best + 5000) % n] = w64[best]
        target = int(rng.integers(0, max(best, 1)))            # an earlier column (or 0)
        if target == best:
            continue
        # W[target] = W[best] with one numerator lowered by 1 where a is +-1 or
        # +-2: the logit drops by 1/1024 or 2/1024, under a bf16 step here
        for kk in np.flatnonzero(np.abs(a_int[i]) <= 2):
            cand = w_int[best].copy()
            step = 1 if a_int[i, kk] > 0 else -1
            if not -14 <= cand[kk] - step <= 14:
                continue
            cand[kk] -= step
            v_best = exact[best] / 1024.0
            v_new = float(a_int[i] @ cand) / 1024.0
            rb = orc.to_f64(orc.round_f64(np.array([v_best, v_new]), "bf16"), "bf16")
            if v_new < v_best and rb[0] == rb[1] and a_int[i, kk] != 0:
                w_int[target] = cand
                w64[target] = cand
                break
    return a_int, w_int


@pytest.mark.parametrize("m,kernel", [(1, None), (8, None), (32, None), (40, None), (32, L.KERNEL_MFMA_STAGED)],
                         ids=["M1", "M8", "M32", "M40-staged", "M32-staged"])
def test_lm_head_exact_inputs_reference_tokens(m, kernel):
    """At the LM-head shape (151936 x 1024) on exact inputs (fp32 logits
    exact in any order), the greedy head's default ranking returns exactly
    the reference's token: the first index of the maximum of the exact
    logits rounded to bf16 (F.linear in bf16, then .float().argmax(-1),
    embed_head.py:61, sampler.py:15, 21), and its bf16 logit; the rows carry
    planted earlier columns that only tie after rounding.  fp32 ranking
    returns the exact fp32 argmax instead."""
    n, k = 151936, 1024
    a_int, w_int = _exact_head_inputs(m, n, k, 400 + m)
    a = torch.from_numpy(a_int.astype(np.float32) / 32).bfloat16()
    w = torch.from_numpy(w_int.astype(np.float32) / 32).bfloat16()
    exact = (a_int.astype(np.float64) @ w_int.T.astype(np.float64)) / 1024.0   # float64, exact
    rounded = orc.to_f64(orc.round_f64(exact, "bf16"), "bf16")
    want = rounded.argmax(-1)                                 # numpy: first index on ties
    want_f32 = exact.argmax(-1)
    assert (want != want_f32).sum() >= max(1, m // 2), "planted near-ties missing"
    ad, wd = a.to(DEV), w.to(DEV)
    _say(f"lm head exact inputs M={m} kernel={kernel}")
    if kernel is None:
        tokens, values = G.gemm_argmax(ad, wd)
        t32, _ = G.gemm_argmax(ad, wd, torch.float32)
    else:
        tokens, values = G.gemm_argmax_with_kernel(ad, wd, kernel)
        t32, _ = G.gemm_argmax_with_kernel(ad, wd, kernel, torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(tokens.cpu().numpy(), want)
    np.testing.assert_array_equal(values.cpu().numpy().astype(np.float64), rounded[np.arange(m), want])
    np.testing.assert_array_equal(t32.cpu().numpy(), want_f32)


@pytest.mark.parametrize("m", [1, 32, 40])
def test_lm_head_random_inputs_match_torch_reference(m):
    """Random Qwen-like inputs at the LM-head shape: the fused greedy head
    against the reference's composition on this GPU (torch's bf16 F.linear,
    then .float().argmax(-1)).  A row whose oracle candidate set (every
    token an fp32 sum within the accumulation bound can give after bf16
    rounding) has one member must give that token on both paths; a row whose
    top logits straddle a rounding boundary within the bound may differ, but
    both tokens must be candidates.  The straddling count is printed."""
    n, k = 151936, 1024
    gen = torch.Generator().manual_seed(500 + m)
    a = torch.randn((m, k), generator=gen).bfloat16()
    w = (torch.randn((n, k), generator=gen) * 0.02).bfloat16()
    ad, wd = a.to(DEV), w.to(DEV)
    _say(f"lm head vs torch M={m}")
    tokens, _ = G.gemm_argmax(ad, wd)
    ref_tokens = torch.nn.functional.linear(ad, wd).float().argmax(-1)
    torch.cuda.synchronize()
    tokens, ref_tokens = tokens.cpu().numpy(), ref_tokens.cpu().numpy()
    a64, w64 = a.double().numpy(), w.double().numpy()
    cand = orc.rounded_greedy_candidates(orc.gemm_f64(a64, w64), orc.abs_products_f64(a64, w64), k, "bf16")
    rows = np.arange(m)
    assert cand[rows, tokens].all() and cand[rows, ref_tokens].all()
    determined = cand.sum(-1) == 1
    np.testing.assert_array_equal(tokens[determined], ref_tokens[determined])
    _say(f"  rows {m}: {int(determined.sum())} determined (equal), {int((~determined).sum())} straddling, "
         f"{int((tokens != ref_tokens).sum())} differing")


# ---------------------------------------------------------------------------
# Sampled LM head (Sampler.forward without logits: greedy rows + Gumbel-max)
# ---------------------------------------------------------------------------
SAMPLE_CASES = ([(L.KERNEL_SPLITK_DECODE, m, n) for m in (1, 5, 32) for n in (1000, 70001)]
                + [(L.KERNEL_MFMA_STAGED, m, 1000) for m in (1, 33, 300)])


def _sample_temps(m, gen):
    t = torch.rand(m, generator=gen) * 1.8 + 0.2
    t[::3] = 0.0                       # greedy rows
    if m > 1:
        t[1] = 1e-10                   # <= 1e-10 in float32: greedy
    return t


@pytest.mark.parametrize("kernel,m,n", SAMPLE_CASES, ids=[f"{L.kernel_name(k)}-M{m}-N{n}" for k, m, n in SAMPLE_CASES])
@pytest.mark.parametrize("din", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("rank", ["model", "f32"])
def test_sample_admissible_against_oracle(kernel, m, n, din, rank):
    """Every token is an admissible winner of the oracle's scores (same
    Philox noise, float64 logits, rounded to the input type when the head
    ranks the model dtype); greedy rows are exactly the greedy head's token
    and logit on the same kernel; a sampled row's score is its token's
    l / T - ln E within the budget."""
    gen = torch.Generator().manual_seed(m * 13 + n)
    k = 256
    a = torch.randn((m, k), generator=gen).to(din)
    w = (torch.randn((n, k), generator=gen) * 0.2).to(din)
    temps = _sample_temps(m, gen)
    seed, offset = 0x5EED0000 + m, (3 << 32) | n
    ad, wd, td = a.to(DEV), w.to(DEV), temps.to(DEV)
    _say(f"sample {L.kernel_name(kernel)} {NAME[din]} M={m} N={n}")
    ldt = None if rank == "model" else torch.float32
    tokens, scores = G.gemm_sample_with_kernel(ad, wd, td, seed, offset, kernel, ldt)
    g_tokens, g_values = G.gemm_argmax_with_kernel(ad, wd, kernel, ldt)
    torch.cuda.synchronize()
    tokens, scores = tokens.cpu().numpy(), scores.cpu().numpy()
    greedy = (temps <= 1e-10).numpy()
    np.testing.assert_array_equal(tokens[greedy], g_tokens.cpu().numpy()[greedy])
    np.testing.assert_array_equal(scores[greedy], g_values.cpu().numpy()[greedy])
    a64, w64 = a.double().numpy(), w.double().numpy()
    r = orc.gemm_f64(a64, w64)
    s = orc.abs_products_f64(a64, w64)
    e = orc.sample_exponential(orc.sample_uniform(m, n, seed, offset))
    ldn = NAME[din] if rank == "model" else "f32"
    ok = orc.sample_token_admissible(tokens, r, s, k, temps.numpy(), e, ldn)
    assert ok.all(), f"rows {np.flatnonzero(~ok)[:8]}"
    rows = np.arange(m)
    if rank == "model":
        # the score of the token lies between its lowest and highest
        # possible rounded-logit scores (plus the fp32 score budget)
        lo, hi = orc.rounded_logit_bounds(r, s, k, ldn)
        sc_lo = orc.sample_scores_f64(lo, temps.numpy(), e)[rows, tokens]
        sc_hi = orc.sample_scores_f64(hi, temps.numpy(), e)[rows, tokens]
        slack = 1e-5 * (1 + np.abs(sc_hi))
        assert ((scores >= sc_lo - slack) & (scores <= sc_hi + slack))[~greedy].all()
    else:
        sc = orc.sample_scores_f64(r, temps.numpy(), e)[rows, tokens]
        np.testing.assert_allclose(scores[~greedy], sc[~greedy], rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("kernel,m", [(L.KERNEL_SPLITK_DECODE, 32), (L.KERNEL_MFMA_STAGED, 64)],
                         ids=["splitk_decode", "mfma_staged"])
def test_sample_noise_is_the_oracles_philox(kernel, m):
    """At a huge temperature the score is -ln E (the logits vanish), so each
    row's token must carry the row's largest uniform u of the oracle's
    Philox stream: pins the device generator, its counter layout and word
    choice bit for bit (64 columns: a wrong word or counter would miss the
    maximum on most rows)."""
    gen = torch.Generator().manual_seed(5)
    n, k = 64, 64
    a = torch.randn((m, k), generator=gen).bfloat16()
    w = (torch.randn((n, k), generator=gen) * 0.1).bfloat16()
    temps = torch.full((m,), 1e30)
    seed, offset = 0xDEADBEEF12345678, 99
    _say(f"sample noise {L.kernel_name(kernel)} M={m}")
    tokens, _ = G.gemm_sample_with_kernel(a.to(DEV), w.to(DEV), temps.to(DEV), seed, offset, kernel)
    torch.cuda.synchronize()
    u = orc.sample_uniform(m, n, seed, offset)
    tokens = tokens.cpu().numpy()
    np.testing.assert_array_equal(u[np.arange(m), tokens], u.max(axis=-1))


def test_sample_distribution():
    """8192 rows with the same logits (exact in bf16: a = e_0, W[j] = l_j e_0)
    draw from softmax(l / T): a chi-square test against the exact
    probabilities, and agreement with the oracle's own draws on >= 99.9% of
    rows (the rest are near-ties of the fp32 score)."""
    from scipy import stats
    logits = torch.tensor([1.0, 0.25, -0.5, 2.0, 0.0, 1.5])
    m, n, k, t = 8192, logits.numel(), 8, 0.75
    a = torch.zeros((m, k))
    a[:, 0] = 1.0
    w = torch.zeros((n, k))
    w[:, 0] = logits
    temps = torch.full((m,), t)
    seed, offset = 77, 5
    _say("sample distribution M=8192")
    tokens, _ = G.gemm_sample(a.bfloat16().to(DEV), w.bfloat16().to(DEV), temps.to(DEV), seed, offset)
    torch.cuda.synchronize()
    tokens = tokens.cpu().numpy()
    z = logits.double().numpy() / np.float64(np.float32(t))
    p = np.exp(z - z.max())
    p /= p.sum()
    counts = np.bincount(tokens, minlength=n)
    assert stats.chisquare(counts, p * m).pvalue > 1e-4, counts
    e = orc.sample_exponential(orc.sample_uniform(m, n, seed, offset))
    want = orc.sample_scores_f64(np.tile(logits.double().numpy(), (m, 1)), temps.numpy(), e).argmax(-1)
    assert float((tokens == want).mean()) >= 0.999


def test_sample_offsets_and_graph_replay():
    """A new offset gives new draws; a call captured in a HIP graph replays
    its own seed and offset (the eager call with the same pair gives the
    same tokens on every replay)."""
    gen = torch.Generator().manual_seed(8)
    m, n, k = 16, 5000, 128
    a = torch.randn((m, k), generator=gen).bfloat16().to(DEV)
    w = (torch.randn((n, k), generator=gen) * 0.05).bfloat16().to(DEV)
    temps = torch.full((m,), 1.0, device=DEV)
    _say("sample offsets and graph")
    t0, _ = G.gemm_sample(a, w, temps, 1, 0)
    t1, _ = G.gemm_sample(a, w, temps, 1, 1)
    t0b, _ = G.gemm_sample(a, w, temps, 1, 0)
    torch.cuda.synchronize()
    assert torch.equal(t0, t0b)
    assert not torch.equal(t0, t1)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        G.gemm_sample(a, w, temps, 1, 7)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        t_static, s_static = G.gemm_sample(a, w, temps, 1, 7)
    for step in range(3):
        graph.replay()
        torch.cuda.synchronize()
        t_eager, s_eager = G.gemm_sample(a, w, temps, 1, 7)
        torch.cuda.synchronize()
        assert torch.equal(t_static, t_eager) and torch.equal(s_static, s_eager), f"replay {step}"


@pytest.mark.parametrize("k", [8, 520, 1024, 1032, 2056, 3584])
def test_gemv_load_unrolls(k):
    """gemv_decode issues 1, 2 or 4 loads per lane together depending on K
    (one per 512-element slice of a row, up to 4); every choice sums in the
    same order and meets the bar, including K that leaves the last trip
    partly empty."""
    n = 777
    gen = torch.Generator().manual_seed(k)
    a = torch.randn((1, k), generator=gen).bfloat16()
    w = (torch.randn((n, k), generator=gen) * 0.1).bfloat16()
    _say(f"gemv unroll K={k}")
    out = G.gemm_with_kernel(a.to(DEV), w.to(DEV), L.KERNEL_GEMV_DECODE, torch.bfloat16)
    torch.cuda.synchronize()
    _check_tolerance(out.cpu(), a, w, L.B_NK, torch.bfloat16)


def test_reference_shape_matrix():
    """bench.py --matrix: the reference's benchmark matrix (its Qwen3.5 shape
    table in fp16 and bf16, deterministic inputs whose products are exact in
    fp32) on every rung it times; each row must hit the exact product."""
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parent.parent)
    if root not in sys.path:
        sys.path.insert(0, root)
    import bench
    _say("reference shape matrix")
    lines = []
    rows = bench.reference_matrix(torch, L, PKG.workloads, emit=lines.append)
    assert len(rows) == 2 * len(PKG.workloads.QWEN35_SHAPES) and len(lines) == len(rows) + 1
    assert lines[0].split(",") == list(rows[0].keys())
    for r in rows:
        assert r["status"] == "PASS", r
        for c in ("direct_max_abs", "staged_max_abs", "dispatch_max_abs", "staged_nk_max_abs", "dispatch_nk_max_abs"):
            assert float(r[c]) == 0.0, (r["label"], c)
        # on B[K,N] the table takes splitk_decode up to M = 32 (M = 64 on N <= 4096), the staged rung above
        mm, nn = int(r["M"]), int(r["N"])
        assert r["dispatch"] == ("splitk_decode" if mm <= 32 or (mm <= 64 and nn <= 4096) else "mfma_staged"), r["label"]
