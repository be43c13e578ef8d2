"""Pins the CPU oracle (oracle/gemm_oracle.py) before it is trusted.

Each check fixes an oracle function by something other than the oracle's
own formula: exact integer arithmetic, values the reference recorded
(cuda_kernels/gemm/results/rtx3060_gemm_matrix.csv), torch / numpy library
routines, hand-worked ties, brute force over representable values, and
planted mistakes that must be caught.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import gemm_oracle as orc

# ---------------------------------------------------------------------------
# Known-answer inputs
# ---------------------------------------------------------------------------


def test_kat_bench_first_values_by_hand():
    # gemm_bench.cu:296-305: a[0] = (3 % 31 - 15)/32 = -12/32; a[1] = (20-15)/32;
    # b[0] = (5 % 29 - 14)/32 = -9/32; b[1] = (16 - 14)/32.
    a = orc.kat_bench_a_int(2, 3)
    b = orc.kat_bench_b_int(3, 2)
    assert a.ravel().tolist()[:2] == [-12, 5]
    assert b.ravel().tolist()[:2] == [-9, 2]
    assert orc.kat_value(a)[0, 0] == np.float32(-12 / 32)


def test_kat_wmma_first_values_by_hand():
    # gemm_wmma.cu:300-311: a[r][k] = ((17r + 13k) % 31 - 15)/32, w[c][k] = ((11c + 7k) % 29 - 14)/32
    a = orc.kat_wmma_a_int(2, 2)
    w = orc.kat_wmma_w_int(2, 2)
    assert a.tolist() == [[-15, -2], [2, 15]]
    assert w.tolist() == [[-14, -7], [-3, 4]]


@pytest.mark.parametrize("gen", ["bench_a", "bench_b", "wmma_a", "wmma_w"])
def test_kat_values_exact_in_half_types(gen):
    ints = {"bench_a": orc.kat_bench_a_int(7, 64), "bench_b": orc.kat_bench_b_int(64, 7),
            "wmma_a": orc.kat_wmma_a_int(7, 64), "wmma_w": orc.kat_wmma_w_int(7, 64)}[gen]
    v = orc.kat_value(ints)
    assert np.all(np.abs(ints) <= 15)
    assert np.array_equal(orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(v)), v)
    assert np.array_equal(v.astype(np.float16).astype(np.float32), v)


# Shapes whose reference rows recorded direct/staged max-abs 0 against cuBLAS
# (rtx3060_gemm_matrix.csv:4-23, all WMMA-capable rows of gemm_bench.cu:45-57).
KAT_SHAPES = [s for s in orc.DEFAULT_SHAPES if orc.supports_wmma(*s[1:])]


@pytest.mark.parametrize("label,m,n,k", [s for s in KAT_SHAPES if s[1] * s[2] * s[3] <= 64 * 7168 * 1024])
def test_kat_bench_fp32_sum_is_exact(label, m, n, k):
    """The fp32-accumulated product of the KAT inputs is exact in any order,
    so the expected output is the exact value (what cuBLAS returned, with
    zero error, in every reference row)."""
    a_int = orc.kat_bench_a_int(m, k)
    b_int = orc.kat_bench_b_int(k, n)
    exact = orc.exact_kat_int(a_int, b_int, "kn")
    assert np.abs(exact).max() < 2 ** 24  # every partial sum fits fp32 exactly
    f32 = orc.kat_value(a_int) @ orc.kat_value(b_int)  # float32 BLAS, its own order
    assert np.array_equal(f32.astype(np.float64) * 1024.0, exact.astype(np.float64))
    f64 = orc.gemm_f64(orc.kat_value(a_int), orc.kat_value(b_int), "kn")
    assert np.array_equal(f64 * 1024.0, exact.astype(np.float64))


def test_kat_wmma_256_cube_exact():
    """gemm_wmma.cu:279-327: 256^3 FP16 case, W[N,K]."""
    a_int = orc.kat_wmma_a_int(256, 256)
    w_int = orc.kat_wmma_w_int(256, 256)
    exact = orc.exact_kat_int(a_int, w_int, "nk")
    f64 = orc.gemm_f64(orc.kat_value(a_int), orc.kat_value(w_int), "nk")
    assert np.array_equal(f64 * 1024.0, exact.astype(np.float64))
    # a few entries by the definition
    for r, c in [(0, 0), (3, 200), (255, 255)]:
        assert exact[r, c] == sum(int(a_int[r, i]) * int(w_int[c, i]) for i in range(256))


def test_kat_tiled_values_match_float32_arithmetic():
    # gemm_tiled.cu:243-248: (i % 19 - 9) * 0.1f evaluated in float32.
    a = orc.kat_tiled_a(127, 65)
    for i in (0, 5, 9, 18, 19, 1000):
        assert a.ravel()[i] == np.float32(np.float32(i % 19 - 9) * np.float32(0.1))
    # The float32 product is not the decimal literal: -9 * 0.1f = -0.90000004.
    assert a.ravel()[0] == np.float32(-0.90000004) and a.ravel()[0] != np.float32(-0.9)


# ---------------------------------------------------------------------------
# Rounding
# ---------------------------------------------------------------------------


def _bits(x):
    return int(orc.f32_to_bf16_bits(np.array([x], dtype=np.float32))[0])


def test_bf16_rne_hand_worked_cases():
    assert _bits(1.0) == 0x3F80
    assert _bits(1.0 + 2.0 ** -8) == 0x3F80          # tie -> even (down)
    assert _bits(1.0 + 3 * 2.0 ** -8) == 0x3F82      # tie -> even (up)
    assert _bits(1.0 + 2.0 ** -8 + 2.0 ** -20) == 0x3F81
    assert _bits(-0.0) == 0x8000
    assert _bits(float("inf")) == 0x7F80
    assert _bits(np.finfo(np.float32).max) == 0x7F80  # rounds past the largest bf16
    nan = _bits(float("nan"))
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        (rng.standard_normal(2000) * 1e-38).astype(np.float32),  # subnormal range
        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 3.0e38], dtype=np.float32),
    ])
    mine = orc.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine, ref)


def _nearest_even(value: Fraction, candidates):
    """Brute-force correct rounding: nearest candidate, ties to even mantissa."""
    best = sorted(candidates, key=lambda c: (abs(Fraction(c[0]) - value), c[1] & 1))
    return best[0][1]


def _bf16_neighbours(x: float):
    f = np.float32(x)
    b = int(orc.f32_to_bf16_bits(np.array([f]))[0])
    out = []
    for bits in (b - 2, b - 1, b, b + 1, b + 2):
        val = float(orc.bf16_bits_to_f32(np.array([bits], dtype=np.uint16))[0])
        out.append((val, bits))
    return out


@pytest.mark.parametrize("x", [
    1.0 + 2.0 ** -8 + 2.0 ** -30,     # double rounding through fp32 would give 1.0
    1.0 + 2.0 ** -8 - 2.0 ** -30,
    -(3.0 + 2.0 ** -7 + 2.0 ** -35),
    0.1, 1.0 / 3.0, 1234.5678, 2.0 ** -130 + 2.0 ** -140,
])
def test_round_f64_bf16_single_rounding(x):
    got = int(orc.round_f64(np.array([x]), "bf16")[0])
    assert got == _nearest_even(Fraction(x), _bf16_neighbours(x))


@pytest.mark.parametrize("x", [1.0 + 2.0 ** -11 + 2.0 ** -40, 1.0 + 2.0 ** -11 - 2.0 ** -40,
                               0.1, 2.0 ** -24 * 1.5 + 2.0 ** -50, 60000.123])
def test_round_f64_f16_single_rounding(x):
    got = orc.round_f64(np.array([x]), "f16")[0]
    h = np.float16(x)
    cands = [(float(v), int(np.array([v], dtype=np.float16).view(np.uint16)[0]))
             for v in (np.nextafter(np.nextafter(h, -np.inf), -np.inf), np.nextafter(h, -np.inf), h,
                       np.nextafter(h, np.inf), np.nextafter(np.nextafter(h, np.inf), np.inf))]
    want = _nearest_even(Fraction(x), cands)
    assert int(np.array([got], dtype=np.float16).view(np.uint16)[0]) == want


def test_naive_double_rounding_is_caught():
    """A planted mistake (RNE to fp32, then RNE to bf16) differs on the
    double-rounding case, so the single-rounding test above has teeth."""
    x = 1.0 + 2.0 ** -8 + 2.0 ** -30
    naive = int(orc.f32_to_bf16_bits(np.array([x], dtype=np.float64).astype(np.float32))[0])
    assert naive != int(orc.round_f64(np.array([x]), "bf16")[0])


# ---------------------------------------------------------------------------
# ULP metrics
# ---------------------------------------------------------------------------


def test_ulp_distance_float_types():
    x = np.array([1.0, -2.5, 0.0, 1e-3], dtype=np.float32)
    nx = np.nextafter(x, np.float32(np.inf))
    assert orc.ulp_distance(x, nx, "f32").tolist() == [1, 1, 1, 1]
    assert orc.ulp_distance(np.float32(0.0), np.float32(-0.0), "f32") == 0
    tiny = np.float32(np.nextafter(np.float32(0), np.float32(1)))
    assert orc.ulp_distance(-tiny, tiny, "f32") == 2
    h = np.array([1.0, -3.0], dtype=np.float16)
    assert orc.ulp_distance(h, np.nextafter(h, np.float16(np.inf)), "f16").tolist() == [1, 1]
    b = orc.f32_to_bf16_bits(np.array([1.0, -1.0], dtype=np.float32))
    assert orc.ulp_distance(b, b + 1, "bf16").tolist() == [1, 1]


def test_ulp_at_matches_spacing():
    r = np.array([1.0, 0.75, 3.0, 1e-3, 6.0e4])
    assert np.array_equal(orc.ulp_at(r, "f32"), np.spacing(r.astype(np.float32)).astype(np.float64))
    assert np.array_equal(orc.ulp_at(r, "f16"), np.spacing(r.astype(np.float16)).astype(np.float64))
    assert orc.ulp_at(np.array([1.0]), "bf16")[0] == 2.0 ** -7
    assert orc.ulp_at(np.array([0.75]), "bf16")[0] == 2.0 ** -8
    assert orc.ulp_at(np.array([0.0]), "bf16")[0] == 2.0 ** -133


# ---------------------------------------------------------------------------
# Reference GEMM and tolerance
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_gemm_f64_matches_torch(layout):
    rng = np.random.default_rng(1)
    a = rng.standard_normal((37, 53))
    b = rng.standard_normal((29, 53)) if layout == "nk" else rng.standard_normal((53, 29))
    ref = torch.from_numpy(a) @ (torch.from_numpy(b).T if layout == "nk" else torch.from_numpy(b))
    assert np.allclose(orc.gemm_f64(a, b, layout), ref.numpy(), rtol=1e-13, atol=1e-13)


def test_gemm_f64_closed_forms():
    a = np.arange(12, dtype=np.float64).reshape(3, 4)
    assert np.array_equal(orc.gemm_f64(a, np.eye(4), "nk"), a)          # identity W
    ones = np.ones((5, 4))
    assert np.array_equal(orc.gemm_f64(a, ones, "nk"), np.repeat(a.sum(1, keepdims=True), 5, axis=1))
    u = np.array([1.0, 2.0, 3.0])
    v = np.array([4.0, 5.0])
    assert np.array_equal(orc.gemm_f64(u[:, None], v[:, None], "nk"), np.outer(u, v))  # K = 1
    kn = np.arange(20, dtype=np.float64).reshape(4, 5)
    assert np.array_equal(orc.gemm_f64(a, kn, "kn"), orc.gemm_f64(a, kn.T, "nk"))


def _fp32_accumulated(a32, w32):
    """A correct kernel: exact products summed in fp32 (sequential order)."""
    acc = np.zeros((a32.shape[0], w32.shape[0]), dtype=np.float32)
    for kk in range(a32.shape[1]):
        acc += a32[:, kk:kk + 1] * w32[:, kk][None, :]
    return acc


def test_tolerance_accepts_fp32_accumulation_and_catches_planted_mistakes():
    gen = torch.Generator().manual_seed(3)
    m, n, k = 16, 48, 1024
    a = (torch.randn((m, k), generator=gen)).to(torch.bfloat16).float().numpy()
    w = (torch.randn((n, k), generator=gen) * 0.02).to(torch.bfloat16).float().numpy()
    a64, w64 = a.astype(np.float64), w.astype(np.float64)
    r = orc.gemm_f64(a64, w64)
    tol = orc.gemm_tolerance(r, orc.abs_products_f64(a64, w64), k, "bf16")

    def ok(out_f32):
        got = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(out_f32)).astype(np.float64)
        return bool((np.abs(got - r) <= tol).all())

    good = _fp32_accumulated(a, w)
    assert ok(good)
    assert ok(np.flip(_fp32_accumulated(a[:, ::-1].copy(), w[:, ::-1].copy()), 0)[::-1])  # other order
    assert not ok(_fp32_accumulated(a[:, :-8], w[:, :-8]))                  # dropped K chunk
    assert not ok(_fp32_accumulated(a, np.roll(w, 1, axis=0)))              # wrong W row
    assert not ok(_fp32_accumulated(a, w[:, ::-1].copy()))                  # reversed K on one operand
    bad = good.copy()
    bad[3, 7] = -bad[3, 7] if abs(bad[3, 7]) > 0.05 else bad[3, 7] + 0.1
    assert not ok(bad)                                                       # one wrong element


def _fp16_down_sample(seed=3, m=48, n=96, k=3584):
    """Inputs of the fp16 down-projection workload's distributions
    (A ~ N(0, 0.5), W ~ N(0, 0.02), K = 3584), rounded to fp16."""
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal((m, k)) * 0.5).astype(np.float16)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    return a, w


def test_narrow_parity_accepts_another_fp32_order():
    """An fp32 GEMM summing K in another order (numpy's float32 BLAS on the
    reversed K axis) is within 2 fp16 ulp of torch's fp32 GEMM rounded once
    on every element but a few cancellations, fewer than the cap."""
    a, w = _fp16_down_sample()
    a64, w64 = a.astype(np.float64), w.astype(np.float64)
    r = orc.gemm_f64(a64, w64)
    s = orc.abs_products_f64(a64, w64)
    other = (a[:, ::-1].astype(np.float32) @ w[:, ::-1].astype(np.float32).T).astype(np.float16)
    ref = (torch.from_numpy(a).float() @ torch.from_numpy(w).float().T).to(torch.float16).numpy()
    stats = orc.narrow_parity(other, ref, r, s, "f16")
    assert stats["ok"].all() and stats["max_ulp_checked"] <= 2
    assert stats["cancel_beyond"] <= orc.cancellation_cap(r.size)


def test_narrow_parity_catches_what_the_fraction_rule_passed():
    """The earlier bar (every element within 2 ulp + the fp32 accumulation
    bound of the float64 product, and >= 99% within 2 ulp of it) passes a
    kernel that mis-rounds 0.5% of the fp16 down-projection outputs by 10
    ulp: the accumulation bound is tens of fp16 ulp at K = 3584.  The
    elementwise bar against the fp32 reference rejects it."""
    a, w = _fp16_down_sample()
    a64, w64 = a.astype(np.float64), w.astype(np.float64)
    r = orc.gemm_f64(a64, w64)
    s = orc.abs_products_f64(a64, w64)
    k = a.shape[1]
    ref = (torch.from_numpy(a).float() @ torch.from_numpy(w).float().T).to(torch.float16).numpy()
    bad = ref.copy()
    tol = orc.gemm_tolerance(r, s, k, "f16")
    # 0.5% of the outputs, among those (three in four) where 10 ulp is still
    # inside the old absolute bound
    rng = np.random.default_rng(0)
    loose = np.flatnonzero((12 * orc.ulp_at(r, "f16") < tol).reshape(-1))
    assert loose.size > 0.5 * bad.size
    idx = rng.choice(loose, size=bad.size // 200, replace=False)
    flat = bad.reshape(-1).view(np.uint16)
    flat[idx] = flat[idx] + 10          # 10 fp16 ulp away (same sign, no overflow at these magnitudes)
    # the old rule passes it
    assert (np.abs(bad.astype(np.float64) - r) <= tol).all()
    assert float((orc.ulp_distance(bad, orc.round_f64(r, "f16"), "f16") <= 2).mean()) >= 0.99
    # the elementwise bar does not: non-cancellation elements beyond 2 ulp,
    # or more cancellation elements than the cap
    stats = orc.narrow_parity(bad, ref, r, s, "f16")
    assert stats["beyond"] >= bad.size // 200
    assert not stats["ok"].all() or stats["cancel_beyond"] > orc.cancellation_cap(bad.size)


def test_cancellation_cap_rejects_a_tenfold_rate():
    """The per-dtype cap rejects a kernel whose cancellation elements go
    beyond 2 ulp ten times as often as the library's (fp16: measured 1 in
    10^4, planted 1 in 1500 of the outputs, all among the cancellation
    elements), which the earlier flat cap of 1 in 1000 let through."""
    a, w = _fp16_down_sample(m=256, n=192)
    a64, w64 = a.astype(np.float64), w.astype(np.float64)
    r = orc.gemm_f64(a64, w64)
    s = orc.abs_products_f64(a64, w64)
    ref = (torch.from_numpy(a).float() @ torch.from_numpy(w).float().T).to(torch.float16).numpy()
    cancel = np.flatnonzero((np.abs(r) <= orc.CANCELLATION * s).reshape(-1))
    planted = ref.size // 1500
    assert cancel.size > 4 * planted
    bad = ref.copy()
    idx = np.random.default_rng(1).choice(cancel, size=planted, replace=False)
    flat = bad.reshape(-1).view(np.uint16)
    flat[idx] = flat[idx] ^ 0x8000       # sign flipped: far beyond 2 ulp unless the value is zero
    stats = orc.narrow_parity(bad, ref, r, s, "f16")
    assert stats["ok"].all()             # every planted element is a cancellation element
    assert stats["cancel_beyond"] >= planted * 9 // 10
    assert stats["cancel_beyond"] <= max(8, ref.size // 1000)            # the flat cap passes it
    assert stats["cancel_beyond"] > orc.cancellation_cap(ref.size, "f16")  # the per-dtype cap does not


def test_narrow_parity_exempts_only_cancellations():
    """An element whose exact value cancels (|r| under 2^-6 of the sum of
    its terms' magnitudes) may exceed 2 ulp (its low bits follow the
    summation order); an ordinary element one step beyond 2 ulp may not."""
    r = np.array([[1e-4, 1.0]])
    scale = np.array([[1.0, 1.0]])
    ref = np.array([[0.0, 1.0]], dtype=np.float16)
    three_up = np.nextafter(np.nextafter(np.nextafter(np.float16(1.0), np.float16(2)), np.float16(2)), np.float16(2))
    got = np.array([[np.float16(1e-4), three_up]], dtype=np.float16)
    stats = orc.narrow_parity(got, ref, r, scale, "f16")
    assert stats["beyond"] == 2 and stats["cancel_beyond"] == 1
    np.testing.assert_array_equal(stats["ok"], [[True, False]])
    assert stats["max_ulp_checked"] == 3
    assert orc.cancellation_cap(100) == 8 and orc.cancellation_cap(10 ** 6) == 500
    assert orc.cancellation_cap(10 ** 6, "bf16") == 33 and orc.cancellation_cap(8388608, "bf16") == 279


def test_rel_frobenius_and_checks():
    ref = np.array([[1.0, 2.0], [3.0, 4.0]])
    assert orc.rel_frobenius(ref, ref) == 0.0
    assert math.isclose(orc.rel_frobenius(ref * 1.001, ref), 1e-3, rel_tol=1e-9)
    assert orc.check_result(ref.astype(np.float32), ref)["correct"]
    assert not orc.check_result(ref.astype(np.float32) + 1e-3, ref)["correct"]
    assert not orc.check_result(np.array([np.nan, 1.0]), np.array([1.0, 1.0]))["correct"]
    cb = orc.compare_bench(np.array([1.0, 2.06]), np.array([1.0, 2.0]))
    assert cb["correct"] and math.isclose(cb["max_absolute"], 0.06, rel_tol=1e-9)
    assert not orc.compare_bench(np.array([1.0, 2.1]), np.array([1.0, 2.0]))["correct"]
    cr = orc.compare_result(np.array([1.0, np.inf, 3.0]), np.array([1.0, 2.0, 3.0]), 1e-2, 1e-2)
    assert cr["non_finite"] == 1 and not cr["correct"]


# ---------------------------------------------------------------------------
# Reference dispatch policy and repeat rule, against the recorded CSV columns
# ---------------------------------------------------------------------------

# (dtype, label) -> (repeats, dispatch), rtx3060_gemm_matrix.csv:2-23
CSV_ROWS = {
    ("fp16", "qwen35_decode_qkv"): (200, "cublas"), ("bf16", "qwen35_decode_qkv"): (200, "cublas"),
    ("fp16", "qwen35_prefill16_qkv"): (99, "cublas"), ("bf16", "qwen35_prefill16_qkv"): (99, "wmma_direct"),
    ("fp16", "qwen35_prefill64_qkv"): (24, "cublas"), ("bf16", "qwen35_prefill64_qkv"): (24, "cublas"),
    ("fp16", "qwen35_prefill256_qkv"): (10, "cublas"), ("bf16", "qwen35_prefill256_qkv"): (10, "cublas"),
    ("fp16", "qwen35_prefill16_out"): (200, "cublas"), ("bf16", "qwen35_prefill16_out"): (200, "cublas"),
    ("fp16", "qwen35_prefill64_out"): (74, "cublas"), ("bf16", "qwen35_prefill64_out"): (74, "cublas"),
    ("fp16", "qwen35_prefill16_gate_up"): (85, "cublas"),
    ("bf16", "qwen35_prefill16_gate_up"): (85, "wmma_direct"),
    ("fp16", "qwen35_prefill64_gate_up"): (21, "cublas"), ("bf16", "qwen35_prefill64_gate_up"): (21, "cublas"),
    ("fp16", "qwen35_prefill64_down"): (42, "cublas"), ("bf16", "qwen35_prefill64_down"): (42, "cublas"),
    ("fp16", "square256"): (200, "cublas"), ("bf16", "square256"): (200, "cublas"),
    ("fp16", "square512"): (74, "cublas"), ("bf16", "square512"): (74, "cublas"),
}


@pytest.mark.parametrize("dtype,label", sorted(CSV_ROWS))
def test_reference_policy_matches_recorded_rows(dtype, label):
    m, n, k = {s[0]: s[1:] for s in orc.DEFAULT_SHAPES}[label]
    repeats, dispatch = CSV_ROWS[(dtype, label)]
    assert orc.repeats_for(2.0 * m * n * k) == repeats
    assert orc.choose_path_reference(m, n, k, dtype) == dispatch


# ---------------------------------------------------------------------------
# Fused SiLU-and-mul oracle
# ---------------------------------------------------------------------------
def test_silu_closed_form_against_torch():
    x = np.concatenate([np.linspace(-60, 60, 4001), [-1000.0, -745.0, 0.0, 745.0, 1000.0]])
    want = torch.nn.functional.silu(torch.from_numpy(x)).numpy()
    got = orc.silu_f64(x)
    np.testing.assert_allclose(got, want, rtol=1e-15, atol=1e-300)
    assert got[-5] == 0.0 and np.signbit(got[-5])      # -1000 * sigmoid(-1000) = -0


def test_silu_slope_bound_brute_force():
    # the propagation term of silu_mul_tolerance relies on |silu'| <= 1.1
    x = np.linspace(-40, 40, 800001)
    slope = np.diff(orc.silu_f64(x)) / np.diff(x)
    assert slope.max() <= orc.SILU_SLOPE_BOUND and slope.max() > 1.099
    assert slope.min() >= -orc.SILU_SLOPE_BOUND


def test_silu_mul_matches_reference_composition():
    """SiluAndMul(x) = F.silu(x[:, :n]) * x[:, n:] of the merged projection
    output (layers/activation.py:8-11), here in float64."""
    rng = np.random.default_rng(5)
    a, w = rng.standard_normal((7, 48)), rng.standard_normal((2 * 20, 48)) * 0.2
    r, g, u = orc.silu_mul_f64(a, w)
    y = torch.from_numpy(a) @ torch.from_numpy(w).T
    x1, x2 = y.chunk(2, -1)
    # numpy and torch sum the float64 products in different orders
    np.testing.assert_allclose(r, (torch.nn.functional.silu(x1) * x2).numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(g, x1.numpy(), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(u, x2.numpy(), rtol=1e-12, atol=1e-13)
    with pytest.raises(ValueError):
        orc.silu_mul_f64(a, w[:-1])


def _fp32_fused(a, w, dtype):
    """What a fused kernel computes: fp32 accumulation, silu and product in
    fp32, one rounding to the output type."""
    n = w.shape[0] // 2
    a32, w32 = torch.from_numpy(a).float(), torch.from_numpy(w).float()
    g, u = a32 @ w32[:n].T, a32 @ w32[n:].T
    out = torch.nn.functional.silu(g) * u
    return out.to(torch.bfloat16 if dtype == "bf16" else torch.float16).double().numpy()


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_silu_mul_tolerance_accepts_fused_and_rejects_planted(dtype):
    rng = np.random.default_rng(9)
    k, n = 512, 96
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    a = torch.from_numpy(rng.standard_normal((33, k))).to(tdt).double().numpy()
    w = torch.from_numpy(rng.standard_normal((2 * n, k)) * 0.1).to(tdt).double().numpy()
    r, g, u = orc.silu_mul_f64(a, w)
    sg = orc.abs_products_f64(a, w[:n])
    su = orc.abs_products_f64(a, w[n:])
    tol = orc.silu_mul_tolerance(r, g, u, sg, su, k, dtype)
    assert (np.abs(_fp32_fused(a, w, dtype) - r) <= tol).all()
    planted = {
        "roles swapped": orc.silu_f64(u) * g,
        "sigmoid without x": g * 0 + u / (1.0 + np.exp(-g)),
        "gate/up rows paired off by one": orc.silu_f64(g) * np.roll(u, 1, axis=1),
        "one K chunk dropped": orc.silu_mul_f64(a[:, 8:], w[:, 8:])[0],
    }
    for name, bad in planted.items():
        assert (np.abs(bad - r) > tol).any(), name


def test_greedy_tokens_first_index_on_ties_and_admissible():
    logits = np.array([[1.0, 3.0, 3.0, -2.0], [0.5, 0.25, 0.5, 0.5]], dtype=np.float32)
    np.testing.assert_array_equal(orc.greedy_tokens(logits), [1, 0])
    np.testing.assert_array_equal(orc.greedy_tokens(logits), torch.from_numpy(logits).argmax(-1).numpy())
    r = logits.astype(np.float64)
    s = np.full_like(r, 1.0)
    k = 1024   # bound = 1024 * 2^-24 = 6.1e-5
    assert orc.greedy_token_admissible(np.array([2, 3]), r, s, k).all()        # ties are admissible
    assert not orc.greedy_token_admissible(np.array([0, 1]), r, s, k).any()    # clearly smaller logits are not


@pytest.mark.parametrize("dtype,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_rounded_greedy_candidates_exact_logits_match_torch(dtype, tdt):
    """With exact logits (zero accumulation bound) there is one candidate
    per row: torch's argmax of the logits converted to the model dtype and
    read back as float32 (the reference's F.linear output and Sampler's
    .float().argmax(-1)).  The logits are float32 values, so torch's
    conversion rounds once.  Many rows hold values that differ in fp32 but
    tie once rounded, where the first index must win."""
    gen = torch.Generator().manual_seed(3)
    base = torch.randn(64, 300, generator=gen) * 3
    # near-ties: copies of each row's best value nudged by less than a
    # rounding step, placed before and after it
    best = base.argmax(-1)
    for i in range(64):
        v = float(base[i, best[i]])
        base[i, (int(best[i]) + 7) % 300] = v * (1 - 2.0 ** -12)
        base[i, (int(best[i]) + 150) % 300] = v * (1 + 2.0 ** -13)
    r32 = base.numpy().astype(np.float32)
    cand = orc.rounded_greedy_candidates(r32.astype(np.float64), np.zeros_like(r32, dtype=np.float64), 1024, dtype)
    assert (cand.sum(-1) == 1).all()
    want = torch.from_numpy(r32).to(tdt).float().argmax(-1).numpy()
    np.testing.assert_array_equal(cand.argmax(-1), want)
    # ranking the fp32 values instead picks another column on some rows
    assert (r32.argmax(-1) != want).any()


def test_first_argmax_candidates_brute_force():
    """Every column the candidate mask admits is reached by its extremal
    assignment (that logit at its top, every other at its bottom), every
    assignment drawn inside the intervals picks an admitted column, and a
    column the mask rejects is never picked."""
    rng = np.random.default_rng(5)
    for trial in range(300):
        n = int(rng.integers(1, 7))
        lo = rng.integers(-4, 5, size=(1, n)).astype(np.float64) / 4
        hi = lo + rng.integers(0, 3, size=(1, n)) / 4
        mask = orc.first_argmax_candidates(lo, hi)[0]
        for j in range(n):
            if mask[j]:
                x = lo[0].copy()
                x[j] = hi[0, j]
                assert int(np.argmax(x)) == j, (lo, hi, j)
        grid = [np.unique(np.concatenate([[lo[0, c], hi[0, c]], np.arange(lo[0, c], hi[0, c], 0.25)]))
                for c in range(n)]
        for _ in range(40):
            x = np.array([rng.choice(g) for g in grid])
            assert mask[int(np.argmax(x))], (lo, hi, x)


def test_rounded_greedy_candidates_catch_planted_mistakes():
    """The tie rule (first index), the rounding type and the accumulation
    bound each change the candidate set on constructed rows."""
    # bf16 spacing at 2.0 is 2^-6: 2.0 and 2.0 + 2^-8 round to the same value
    r = np.array([[1.0, 2.0, 2.0 + 2.0 ** -8, -1.0]])
    s = np.zeros_like(r)
    cand = orc.rounded_greedy_candidates(r, s, 1024, "bf16")
    np.testing.assert_array_equal(cand[0], [False, True, False, False])     # first index of the tie
    last_index = np.flatnonzero(orc.to_f64(orc.round_f64(r, "bf16"), "bf16")[0] == 2.0)[-1]
    assert not cand[0, last_index]                                            # the last-index rule would differ
    cand16 = orc.rounded_greedy_candidates(r, s, 1024, "f16")                # f16 resolves the pair
    np.testing.assert_array_equal(cand16[0], [False, False, True, False])
    # a bound wide enough to cross a rounding boundary admits the other column
    wide = orc.rounded_greedy_candidates(r, np.full_like(r, 1.0e3), 1024, "bf16")   # bound 0.061
    assert wide[0, 1] and wide[0, 2]


def test_sample_admissibility_rounded_logits():
    """With model-dtype logits a column whose exact score is slightly lower
    but whose rounded logit ties the best is admissible; one a full rounding
    step below is not."""
    r = np.array([[0.0, 2.0 + 2.0 ** -8, 2.0, 2.0 - 2.0 ** -5]])
    s = np.zeros_like(r)
    temps = np.array([0.5], dtype=np.float32)
    e = np.ones_like(r)
    assert orc.sample_token_admissible(np.array([2]), r, s, 1024, temps, e, "bf16").all()
    assert not orc.sample_token_admissible(np.array([2]), r, s, 1024, temps, e).any()    # fp32 ranking
    assert not orc.sample_token_admissible(np.array([3]), r, s, 1024, temps, e, "bf16").any()


# ---------------------------------------------------------------------------
# Sampled LM head: Philox noise and the Gumbel-max form of Sampler.forward
# ---------------------------------------------------------------------------
# Known-answer vectors of Philox4x32-10 published with its authors' Random123
# library (kat_vectors: counter, key, expected output).
PHILOX_KATS = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KATS)
def test_philox_known_answers(ctr, key, want):
    got = orc.philox4x32_10(np.array([ctr], dtype=np.uint64), key)[0]
    assert tuple(int(x) for x in got) == want


def test_sample_uniform_layout():
    """u[i, j] comes from word j % 4 of the draw at counter (j // 4, i,
    offset, offset >> 32) under key (seed, seed >> 32), lies in (0, 1] and is
    a multiple of 2^-24."""
    seed, offset = 0x0123456789ABCDEF, (7 << 32) | 5
    u = orc.sample_uniform(3, 9, seed, offset)
    assert ((u > 0) & (u <= 1)).all()
    assert np.array_equal(u * 2.0 ** 24, np.round(u * 2.0 ** 24))
    for i in range(3):
        for j in range(9):
            w = orc.philox4x32_10(np.array([[j // 4, i, 5, 7]], dtype=np.uint64), (0x89ABCDEF, 0x01234567))[0]
            assert u[i, j] == ((int(w[j % 4]) >> 8) + 1) / 2.0 ** 24
    # different offsets and seeds give different draws
    assert not np.array_equal(u, orc.sample_uniform(3, 9, seed, offset + 1))
    assert not np.array_equal(u, orc.sample_uniform(3, 9, seed + 1, offset))


def test_gumbel_scores_pick_the_reference_sample():
    """argmax_j (l / T - ln E) is the reference's argmax_j softmax(l / T) / E
    for the same noise E, on sampled and greedy rows alike."""
    rng = np.random.default_rng(11)
    logits = rng.normal(0.0, 3.0, size=(64, 50))
    temps = rng.uniform(0.05, 2.0, size=64).astype(np.float32)
    temps[::7] = 0.0                      # greedy rows
    temps[3] = np.float32(1e-10)          # <= 1e-10 in float32: greedy
    temps[4] = np.float32(1.2e-10)        # just above: sampled
    e = orc.sample_exponential(orc.sample_uniform(64, 50, 3, 0))
    want = orc.sampler_reference_f64(logits, temps, e)
    got = orc.sample_scores_f64(logits, temps, e).argmax(axis=-1)
    np.testing.assert_array_equal(got, want)
    greedy_rows = temps <= np.float32(1e-10)
    np.testing.assert_array_equal(got[greedy_rows], logits[greedy_rows].argmax(-1))


def _chi2_pvalue(counts: np.ndarray, probs: np.ndarray) -> float:
    from scipy import stats
    expected = probs * counts.sum()
    return float(stats.chisquare(counts, expected).pvalue)


def test_sampled_rows_follow_softmax():
    """20000 rows with the same logits, each with its own noise (the row
    enters the counter), draw from softmax(l / T): a chi-square test against
    the exact probabilities passes, and planted mistakes in the score (+ln E,
    T applied twice, the noise of column j + 1) fail it."""
    logits = np.array([1.0, 0.2, -0.5, 2.0, 0.0, 1.5])
    t = 0.8
    m = 20000
    r = np.tile(logits, (m, 1))
    temps = np.full(m, t, dtype=np.float32)
    e = orc.sample_exponential(orc.sample_uniform(m, logits.size, 2024, 17))
    z = logits / np.float64(np.float32(t))
    p = np.exp(z - z.max())
    p /= p.sum()
    tokens = orc.sample_scores_f64(r, temps, e).argmax(-1)
    assert _chi2_pvalue(np.bincount(tokens, minlength=logits.size), p) > 1e-3
    zz = r / np.float64(np.float32(t))
    planted = {
        "+ln E": (zz + np.log(e)).argmax(-1),
        "T twice": (zz / t - np.log(e)).argmax(-1),
        "no noise": zz.argmax(-1),
    }
    for name, bad in planted.items():
        assert _chi2_pvalue(np.bincount(bad, minlength=logits.size), p) < 1e-6, name


def test_sample_admissibility():
    """The exact winner is admissible; a clearly worse column is not; a
    column whose score is within the fp32 budget of the best is."""
    r = np.array([[0.0, 1.0, 3.0, 2.0]])
    s = np.ones_like(r)
    temps = np.array([0.5], dtype=np.float32)
    e = np.array([[1.0, 1.0, 1.0, 1.0]])
    assert orc.sample_token_admissible(np.array([2]), r, s, 1024, temps, e).all()
    assert not orc.sample_token_admissible(np.array([3]), r, s, 1024, temps, e).any()
    e2 = np.array([[1.0, 1.0, 1.0, np.exp(-1.0 + 1e-7)]])   # column 3 scores 4 + 1 - 1e-7 against 6
    assert not orc.sample_token_admissible(np.array([3]), r, s, 1024, temps, e2).any()
    e3 = np.array([[1.0, 1.0, 1.0, np.exp(-2.0 + 1e-6)]])   # column 3 within 1e-6 of column 2
    assert orc.sample_token_admissible(np.array([3]), r, s, 1024, temps, e3).all()


# ---------------------------------------------------------------------------
# Prologues: output gate and residual add + RMSNorm
# ---------------------------------------------------------------------------
def _bf16(x) -> np.ndarray:
    return orc.encode(np.asarray(x, dtype=np.float32), "bf16")


def test_sigmoid_closed_forms_and_torch():
    x = np.concatenate([np.linspace(-40, 40, 8001), [-800.0, 0.0, 800.0]])
    got = orc.sigmoid_f64(x)
    np.testing.assert_allclose(got, torch.sigmoid(torch.from_numpy(x)).numpy(), rtol=1e-15, atol=1e-300)
    assert orc.sigmoid_f64(np.array([0.0]))[0] == 0.5
    np.testing.assert_allclose(got + orc.sigmoid_f64(-x), 1.0, rtol=0, atol=1e-15)   # sigma(-x) = 1 - sigma(x)


def test_gate_view_is_the_chunk_of_q_proj():
    """gate_view reads q_proj(x).view(-1, H, 2D).chunk(2, -1)[1]
    (qwen3_5.py:81-86) out of the un-chunked rows."""
    m, heads, d = 3, 4, 8
    q = torch.arange(m * heads * 2 * d, dtype=torch.float64).view(m, heads, 2 * d)
    want = q.chunk(2, dim=-1)[1].reshape(m, heads * d).numpy()
    got = orc.gate_view(q.view(m, -1).numpy()[:, d:], heads * d, d, 2 * d)
    np.testing.assert_array_equal(got, want)


def test_sigmoid_gate_closed_forms():
    a = _bf16([[3.0, -5.5, 0.375, 1e-3]])
    half = orc.to_f64(orc.sigmoid_gate(a, _bf16([[0.0] * 4]), "bf16"), "bf16")
    np.testing.assert_array_equal(half, orc.to_f64(a, "bf16") / 2)      # sigmoid(0) = 1/2 exactly
    one = orc.to_f64(orc.sigmoid_gate(a, _bf16([[60.0] * 4]), "bf16"), "bf16")
    np.testing.assert_array_equal(one, orc.to_f64(a, "bf16"))           # sigmoid(60) rounds to 1


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_sigmoid_gate_matches_torch_two_ops(dtype):
    """`output * torch.sigmoid(gate)` (qwen3_5.py:95) run by torch on the CPU
    in the element type: equal to the oracle except where fp32 and float64
    sigmoids round differently next to a tie (<= 1 ulp, rare); a single
    rounding of a * sigmoid(g) (a planted mistake) differs far more often."""
    rng = np.random.default_rng(17)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    a = torch.from_numpy(rng.standard_normal((64, 512))).to(tdt)
    g = torch.from_numpy(rng.standard_normal((64, 512)) * 4).to(tdt)
    ref = a * torch.sigmoid(g)
    store = (lambda t: t.view(torch.int16).numpy().view(np.uint16)) if dtype == "bf16" else (lambda t: t.numpy())
    want = orc.sigmoid_gate(store(a), store(g), dtype)
    ulps = orc.ulp_distance(store(ref), want, dtype)
    assert ulps.max() <= 1 and float((ulps == 0).mean()) >= 0.999
    single = orc.round_f64(a.double().numpy() * orc.sigmoid_f64(g.double().numpy()), dtype)
    assert float((orc.ulp_distance(single, want, dtype) != 0).mean()) > 0.01


def test_add_norm_operand_and_scale_by_hand():
    h = _bf16([[1.5, 2.0, -3.0, 0.25]])
    r = _bf16([[0.5, -1.0, 1.0, 0.25]])
    w = _bf16([0.0, 1.0, -0.5, 0.0])
    s, y, res = orc.add_norm_operand(h, r, w, "bf16")
    np.testing.assert_array_equal(s, [[2.0, 1.0, -2.0, 0.5]])
    np.testing.assert_array_equal(orc.to_f64(y, "bf16"), [[2.0, 2.0, -1.0, 0.5]])        # s (1 + w)
    np.testing.assert_array_equal(orc.to_f64(res, "bf16"), s)
    assert orc.norm_scale_f64(s, 0.0)[0] == 1.0 / math.sqrt((4 + 1 + 4 + 0.25) / 4)
    # constant rows and an all-zero row (only eps is left)
    np.testing.assert_allclose(orc.norm_scale_f64(np.full((1, 64), 3.0), 1e-6), 1 / math.sqrt(9 + 1e-6), rtol=1e-15)
    assert orc.norm_scale_f64(np.zeros((1, 8)), 1e-6)[0] == 1.0 / math.sqrt(1e-6)


def test_add_norm_operand_order_needs_bf16_range():
    """Why the fused norm takes bf16 only: its operand s (1 + w) is rounded
    before the row scale.  With |s| ~ 2e4 and 1 + w = 4 that is 8e4, beyond
    fp16's 65504, and a row of s ~ 1e-6 lands in fp16's subnormals, while the
    reference's operand s rsqrt(mean s^2 + eps) (1 + w) (layernorm.py:126-130)
    is a finite, normal fp16 number on both rows.  In bf16 (fp32's exponent range) both orders stay
    finite and normal."""
    s = np.array([[2.0e4, -1.5e4, 1.0e4, 2.0e4], [1.0e-6, -2.0e-6, 1.5e-6, 1.0e-6]], dtype=np.float32)
    w = np.full(4, 3.0, dtype=np.float32)                       # 1 + w = 4
    zero = np.zeros_like(s)
    _, y16, _ = orc.add_norm_operand(s.astype(np.float16), zero.astype(np.float16), w.astype(np.float16), "f16")
    assert np.isinf(orc.to_f64(y16[0], "f16")).any()              # overflow on the large row
    tiny = np.abs(orc.to_f64(y16[1], "f16"))
    assert (tiny < 2.0 ** -14).all() and (tiny > 0).all()         # subnormal on the small row
    ref = s.astype(np.float64) * orc.norm_scale_f64(s, 1e-6)[:, None] * 4.0
    assert (np.abs(ref) >= 2.0 ** -14).all() and (np.abs(ref) < 65504).all()   # normal, finite fp16
    _, yb, _ = orc.add_norm_operand(orc.encode(s, "bf16"), orc.encode(zero, "bf16"), orc.encode(w, "bf16"), "bf16")
    yb64 = np.abs(orc.to_f64(yb, "bf16"))
    assert np.isfinite(yb64).all() and (yb64 >= 2.0 ** -126).all()


def test_add_norm_residual_matches_reference_and_gemm_close():
    """Qwen3_5RMSNorm.forward(h, residual) in torch (layernorm.py:131-142):
    the new residual is the oracle's bit for bit; normalized @ W^T of the
    reference (rounded after scaling) and scale * (operand @ W^T) of the
    kernels (rounded before) differ by the two roundings only."""
    rng = np.random.default_rng(3)
    k = 256
    h = torch.from_numpy(rng.standard_normal((8, k))).bfloat16()
    r = torch.from_numpy(rng.standard_normal((8, k))).bfloat16()
    w_norm = torch.from_numpy(rng.standard_normal(k) * 0.1).bfloat16()
    summed = h.float() + r.float()
    ref_res = summed.to(torch.bfloat16)
    normalized = (summed * torch.rsqrt(summed.pow(2).mean(-1, keepdim=True) + 1e-6)
                  * (1.0 + w_norm.float())).to(torch.bfloat16)
    st = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    s64, y, res = orc.add_norm_operand(st(h), st(r), st(w_norm), "bf16")
    np.testing.assert_array_equal(res, st(ref_res))
    scale = orc.norm_scale_f64(s64, 1e-6)
    W = rng.standard_normal((64, k)) * 0.05
    ours = scale[:, None] * (orc.to_f64(y, "bf16") @ W.T)
    theirs = normalized.double().numpy() @ W.T
    bound = 2.0 ** -7 * scale[:, None] * (np.abs(orc.to_f64(y, "bf16")) @ np.abs(W).T)
    assert (np.abs(ours - theirs) <= bound).all()


def test_add_norm_tolerance_accepts_fp32_kernel_and_rejects_planted():
    """An fp32 evaluation of the kernels' formula (fp32 sums, fp32 row scale,
    one rounding) meets add_norm_gemm_tolerance; the plausible mistakes do
    not: residual dropped, w used instead of 1 + w, eps ignored, mean over
    a padded K, the scale applied twice."""
    rng = np.random.default_rng(23)
    k, n, eps = 512, 96, 1e-6
    h = _bf16(rng.standard_normal((24, k)))
    r = _bf16(rng.standard_normal((24, k)))
    tiny = _bf16(rng.standard_normal((2, k)) * 1e-3)
    h[:2], r[:2] = tiny, tiny                            # rows where eps matters
    w_norm = _bf16(rng.standard_normal(k) * 0.1)
    W = orc.to_f64(_bf16(rng.standard_normal((n, k)) * 0.05), "bf16")
    s64, y, _ = orc.add_norm_operand(h, r, w_norm, "bf16")
    y64 = orc.to_f64(y, "bf16")
    scale = orc.norm_scale_f64(s64, eps)
    want = scale[:, None] * (y64 @ W.T)
    tol = orc.add_norm_gemm_tolerance(want, np.abs(y64) @ np.abs(W).T, scale, k, "f32")
    s32 = s64.astype(np.float32)
    ss = (s32 * s32).sum(axis=1, dtype=np.float32)
    scale32 = (np.float32(1.0) / np.sqrt(ss / np.float32(k) + np.float32(eps))).astype(np.float32)
    fp32 = (y64.astype(np.float32) @ W.astype(np.float32).T) * scale32[:, None]
    assert (np.abs(fp32.astype(np.float64) - want) <= tol).all()

    def gemm_with(s_rows, one_w, eps_, k_mean):
        y_ = orc.to_f64(_bf16((s_rows * one_w).astype(np.float32)), "bf16")
        sc = 1.0 / np.sqrt((s_rows ** 2).sum(axis=1) / k_mean + eps_)
        return sc[:, None] * (y_ @ W.T)
    one_w = 1.0 + orc.to_f64(w_norm, "bf16")
    h64 = orc.to_f64(h, "bf16")
    planted = {
        "residual dropped": gemm_with(h64, one_w, eps, k),
        "w instead of 1 + w": gemm_with(s64, one_w - 1.0, eps, k),
        "eps ignored": gemm_with(s64, one_w, 0.0, k),
        "mean over K + 8": gemm_with(s64, one_w, eps, k + 8),
        "scale applied twice": want * scale[:, None],
    }
    for name, bad in planted.items():
        assert (np.abs(bad - want) > tol).any(), name
