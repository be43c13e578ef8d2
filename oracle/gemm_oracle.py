"""CPU oracle for the shape-aware GEMM path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
torch op, the selection table) imports or calls this module; only tests/,
``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may use it,
and only to check results.

It restates, in numpy, what the reference computes on the CPU for this
path (paths relative to the reference repo):

  * known-answer input generators
      gemm_bench.cu:296-305   a[i]=((17i+3)%31-15)/32, b[i]=((11i+5)%29-14)/32, B[K,N]
      gemm_wmma.cu:300-311    a[r][k]=((17r+13k)%31-15)/32, w[c][k]=((11c+7k)%29-14)/32, W[N,K]
      gemm_tiled.cu:243-248   a[i]=(i%19-9)*0.1f, b[i]=(i%13-6)*0.1f (also gemm.cu:21-22)
  * the double-accumulated reference GEMM (gemm.cu:23-29, gemm_tiled.cu:251-260,
    gemm_wmma.cu:315-327), here in float64 with one final rounding to the
    output type;
  * round-to-nearest-even to bf16 / fp16 (TypeTraits::convert,
    gemm_bench.cu:59-78, which calls __float2bfloat16 / __float2half);
  * the differential checks: compare (gemm_bench.cu:225-250),
    compare_result (gemm_wmma.cu:209-247), check_result (common.cuh:18-31);
  * the dispatch policy supports_wmma / choose_path (gemm_bench.cu:252-273),
    the shape table kDefaultShapes (gemm_bench.cu:45-57) and the repeat
    rule (gemm_bench.cu:371-379);
  * next to the GEMM (nanovllm/): SiluAndMul (layers/activation.py:8-11),
    the sampler (layers/sampler.py:8-21: greedy argmax, and the sampled
    rows' argmax of softmax(l / T) / E with E ~ Exp(1), here with the noise
    of the library's counter-based generator, Philox4x32-10), the output gate
    of gated attention (models/qwen3_5.py:95) and the residual add +
    zero-centred RMSNorm (layers/layernorm.py:131-142).

Pinning (what fixes each function independently of this file): the KAT
results are checked against exact integer arithmetic and against the
reference's recorded zero error on every KAT row
(results/rtx3060_gemm_matrix.csv:4-23); the float64 GEMM against
torch.matmul in float64; the bf16/fp16 rounding against torch's and numpy's
conversions and against hand-picked ties; the ULP metric against
np.nextafter; Philox4x32-10 against the published known-answer vectors of
its authors' Random123 distribution, and the sampled-row score
l / T - ln E against the reference's softmax(l / T) / E (same argmax) and
against the distribution it must draw from.  See tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# Known-answer generators
# ---------------------------------------------------------------------------

def kat_bench_a_int(m: int, k: int) -> np.ndarray:
    """Numerators (units of 1/32) of A[M,K] from gemm_bench.cu:296-300."""
    i = np.arange(m * k, dtype=np.int64)
    return ((i * 17 + 3) % 31 - 15).reshape(m, k)


def kat_bench_b_int(k: int, n: int) -> np.ndarray:
    """Numerators of B[K,N] (row-major, flat index i) from gemm_bench.cu:301-305."""
    i = np.arange(k * n, dtype=np.int64)
    return ((i * 11 + 5) % 29 - 14).reshape(k, n)


def kat_wmma_a_int(m: int, k: int) -> np.ndarray:
    """Numerators of A[M,K] from gemm_wmma.cu:300-305."""
    r = np.arange(m, dtype=np.int64)[:, None]
    kk = np.arange(k, dtype=np.int64)[None, :]
    return (r * 17 + kk * 13) % 31 - 15


def kat_wmma_w_int(n: int, k: int) -> np.ndarray:
    """Numerators of W[N,K] (B col-major) from gemm_wmma.cu:306-311."""
    c = np.arange(n, dtype=np.int64)[:, None]
    kk = np.arange(k, dtype=np.int64)[None, :]
    return (c * 11 + kk * 7) % 29 - 14


def kat_value(numerators: np.ndarray) -> np.ndarray:
    """numerator * 0.03125 as float32 (exact: |value| <= 15/32)."""
    return numerators.astype(np.float32) * np.float32(0.03125)


def kat_tiled_a(m: int, k: int) -> np.ndarray:
    """A[M,K] fp32 from gemm_tiled.cu:243-245 / gemm.cu:21: (i%19-9)*0.1f."""
    i = np.arange(m * k, dtype=np.int64)
    return ((i % 19 - 9).astype(np.float32) * np.float32(0.1)).reshape(m, k)


def kat_tiled_b(k: int, n: int) -> np.ndarray:
    """B[K,N] fp32 from gemm_tiled.cu:246-248 / gemm.cu:22: (i%13-6)*0.1f."""
    i = np.arange(k * n, dtype=np.int64)
    return ((i % 13 - 6).astype(np.float32) * np.float32(0.1)).reshape(k, n)


# ---------------------------------------------------------------------------
# bf16 / fp16 encodings (bf16 is carried as uint16 bit patterns)
# ---------------------------------------------------------------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even; NaN -> quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    quiet = ((u >> 16) | 0x40) & 0xFFFF
    return np.where(nan, quiet, rounded).astype(np.uint16)


def f64_to_f32_round_odd(x: np.ndarray) -> np.ndarray:
    """float64 -> float32 rounded to odd (truncate, then set the last bit if
    inexact).  A second rounding of this value to any format with at least
    2 fewer significand bits equals one correct rounding of x."""
    x = np.asarray(x, dtype=np.float64)
    f = x.astype(np.float32)
    back = f.astype(np.float64)
    inexact = back != x
    bits = f.view(np.uint32).copy()
    over = inexact & (np.abs(back) > np.abs(x))
    bits[over] -= 1
    bits[inexact] |= 1
    return bits.view(np.float32)


def round_f64(x: np.ndarray, out: str) -> np.ndarray:
    """One correct round-to-nearest-even of float64 values to `out`.

    Returns float32 / float16 arrays, or uint16 bf16 bit patterns."""
    x = np.asarray(x, dtype=np.float64)
    if out == "f32":
        return x.astype(np.float32)
    if out == "f16":
        return f64_to_f32_round_odd(x).astype(np.float16)
    if out == "bf16":
        return f32_to_bf16_bits(f64_to_f32_round_odd(x))
    raise ValueError(out)


def to_f64(values: np.ndarray, dtype: str) -> np.ndarray:
    """Decode an array of `dtype` ("f32", "f16", or "bf16" bits) to float64."""
    if dtype == "bf16":
        return bf16_bits_to_f32(values).astype(np.float64)
    return np.asarray(values).astype(np.float64)


def encode(x_f32: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> storage of `dtype` with round-to-nearest-even."""
    if dtype == "f32":
        return np.asarray(x_f32, dtype=np.float32)
    if dtype == "f16":
        return np.asarray(x_f32, dtype=np.float32).astype(np.float16)
    if dtype == "bf16":
        return f32_to_bf16_bits(x_f32)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# Reference GEMM
# ---------------------------------------------------------------------------

def gemm_f64(a64: np.ndarray, b64: np.ndarray, b_layout: str = "nk") -> np.ndarray:
    """C = A * B in float64 (gemm.cu:23-29): B is W[N,K] for "nk", B[K,N] for "kn"."""
    a64 = np.asarray(a64, dtype=np.float64)
    b64 = np.asarray(b64, dtype=np.float64)
    if b_layout == "nk":
        return a64 @ b64.T
    if b_layout == "kn":
        return a64 @ b64
    raise ValueError(b_layout)


def abs_products_f64(a64: np.ndarray, b64: np.ndarray, b_layout: str = "nk") -> np.ndarray:
    """S[m,n] = sum_k |A[m,k] B(k,n)|, the scale of fp32 accumulation error."""
    return gemm_f64(np.abs(a64), np.abs(b64), b_layout)


def exact_kat_int(a_int: np.ndarray, b_int: np.ndarray, b_layout: str = "nk") -> np.ndarray:
    """Exact integer numerators (units of 1/1024) of a KAT product."""
    a_int = np.asarray(a_int, dtype=np.int64)
    b_int = np.asarray(b_int, dtype=np.int64)
    return a_int @ (b_int.T if b_layout == "nk" else b_int)


# ---------------------------------------------------------------------------
# Error metrics
# ---------------------------------------------------------------------------
_FMT = {"f32": (32, 23, 127), "f16": (16, 10, 15), "bf16": (16, 7, 127)}


def ulp_at(r64: np.ndarray, dtype: str) -> np.ndarray:
    """Spacing of `dtype` at |r| (the subnormal spacing below the smallest normal)."""
    _, mant, bias = _FMT[dtype]
    r = np.abs(np.asarray(r64, dtype=np.float64))
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(r > 0, r, 1.0)))
    e = np.maximum(np.where(r > 0, e, 1 - bias), 1 - bias)
    return np.ldexp(1.0, (e - mant).astype(np.int64))


def _ordered(bits: np.ndarray, nbits: int) -> np.ndarray:
    b = np.asarray(bits).astype(np.int64)
    sign = (b >> (nbits - 1)) & 1
    mag = b & ((1 << (nbits - 1)) - 1)
    return np.where(sign == 1, -mag, mag)


def ulp_distance(x: np.ndarray, y: np.ndarray, dtype: str) -> np.ndarray:
    """Number of representable `dtype` values between x and y (same encoding
    as `encode`/`round_f64` output).  +0 and -0 are the same point."""
    if dtype == "f32":
        xb = np.asarray(x, dtype=np.float32).view(np.uint32)
        yb = np.asarray(y, dtype=np.float32).view(np.uint32)
        return np.abs(_ordered(xb, 32) - _ordered(yb, 32))
    if dtype == "f16":
        xb = np.asarray(x, dtype=np.float16).view(np.uint16)
        yb = np.asarray(y, dtype=np.float16).view(np.uint16)
    else:
        xb = np.asarray(x, dtype=np.uint16)
        yb = np.asarray(y, dtype=np.uint16)
    return np.abs(_ordered(xb, 16) - _ordered(yb, 16))


def fp32_accumulation_bound(s64: np.ndarray, k: int) -> np.ndarray:
    """First-order bound K * 2^-24 * sum|a b| on the error of summing K
    exact fp32 products in any order (Higham, gamma_K)."""
    return k * 2.0 ** -24 * np.asarray(s64, dtype=np.float64)


def gemm_tolerance(r64: np.ndarray, s64: np.ndarray, k: int, dtype: str, ulps: float = 2.0) -> np.ndarray:
    """Per-element bound used by the parity tests for narrow and fp32 outputs:
    `ulps` units in the last place of the output type at the exact value,
    plus the fp32 accumulation bound.  Any kernel that accumulates in fp32
    and rounds once to the output type meets it; a dropped or repeated
    K-chunk, a transposed operand or a wrong row exceeds it."""
    return ulps * ulp_at(r64, dtype) + fp32_accumulation_bound(s64, k)


CANCELLATION = 2.0 ** -6


def narrow_parity(got: np.ndarray, ref32: np.ndarray, r64: np.ndarray, scale64: np.ndarray, dtype: str,
                  ulps: int = 2) -> dict:
    """The elementwise bar for bf16 / fp16 outputs: every element within
    `ulps` units of the fp32-accumulated reference rounded once (`ref32`,
    encoded like `got`).  Two fp32 sums of the same products in different
    orders differ by a few fp32 ulps of their terms, which is far below an
    output ulp unless the exact value r cancels: |r| <= 2^-6 scale, scale
    the sum of the magnitudes of the terms (sum_k |a w| for a GEMM), where
    the low output bits are decided by the summation order.  Only such
    elements may exceed `ulps` (callers hold them to the absolute fp32
    accumulation bound and cap their number).  Returns {"ok": mask,
    "beyond": elements beyond `ulps`, "cancel_beyond": of those, the
    cancellation elements, "max_ulp": over all elements, "max_ulp_checked":
    over the non-cancellation ones, "within": fraction within `ulps`}."""
    d = ulp_distance(got, ref32, dtype)
    cancel = np.abs(np.asarray(r64, dtype=np.float64)) <= CANCELLATION * np.asarray(scale64, dtype=np.float64)
    beyond = d > ulps
    checked = d[~cancel]
    return {"ok": ~beyond | cancel, "beyond": int(beyond.sum()), "cancel_beyond": int((beyond & cancel).sum()),
            "max_ulp": int(d.max()) if d.size else 0,
            "max_ulp_checked": int(checked.max()) if checked.size else 0,
            "within": float((~beyond).mean()) if d.size else 1.0}


def cancellation_cap(size: int, dtype: str = "f16") -> int:
    """How many cancellation elements of `size` outputs may exceed the ULP
    bar: about five times the rate measured on the library's kernels, at
    least 8.  bf16 outputs: 1 in 30000 (measured 53 of 8.39 M on the
    2048 x 4096 x 1024 prefill, 41 of 8.61 M on the row-scaled 2100 x 4100
    GEMM after the add + RMSNorm prologue, at most 2 on any smaller shape);
    fp16 outputs: 1 in 2000 (measured 400 of 4.19 M on the 4096 x 1024 x 3584
    down projection, up to 10 of 65536 on small-M K = 2048 shapes), fp16's
    near-zero outputs sitting in its subnormal range, where one fp32
    rounding of a term is several output ulps."""
    rate = 30000 if dtype == "bf16" else 2000
    return max(8, size // rate)


def rel_frobenius(x: np.ndarray, ref: np.ndarray) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(x - ref) / np.linalg.norm(ref))


def compare_bench(actual: np.ndarray, reference: np.ndarray) -> dict:
    """gemm_bench.cu:225-250: max/mean abs error; FAIL if non-finite or
    |e| > 5e-2 + 1e-2 |ref|."""
    a = np.asarray(actual, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    err = np.abs(a - r)
    bad = ~np.isfinite(a) | (err > 5.0e-2 + 1.0e-2 * np.abs(r))
    return {"max_absolute": float(np.nanmax(err)) if err.size else 0.0,
            "mean_absolute": float(np.nanmean(err)) if err.size else 0.0,
            "correct": not bool(bad.any())}


def compare_result(actual: np.ndarray, reference: np.ndarray, atol: float, rtol: float) -> dict:
    """gemm_wmma.cu:217-247: non-finite count, max/mean abs, rmse over the
    finite elements; FAIL on any non-finite or |e| > atol + rtol |ref|."""
    a = np.asarray(actual, dtype=np.float64)
    r = np.asarray(reference, dtype=np.float64)
    finite = np.isfinite(a)
    err = np.abs(a[finite] - r[finite])
    n = a.size
    return {
        "max_absolute": float(err.max()) if err.size else 0.0,
        "mean_absolute": float(err.sum() / n) if n else 0.0,
        "rmse": float(np.sqrt((err ** 2).sum() / n)) if n else 0.0,
        "non_finite": int((~finite).sum()),
        "correct": bool(finite.all()) and not bool((err > atol + rtol * np.abs(r[finite])).any()),
    }


def check_result(result: np.ndarray, reference: np.ndarray) -> dict:
    """common.cuh:18-31: FAIL if non-finite or |e| > 1e-4 + 1e-4 |ref|."""
    x = np.asarray(result, dtype=np.float32)
    r = np.asarray(reference, dtype=np.float32)
    err = np.abs(x - r)
    ok = np.isfinite(x).all() and not (err > np.float32(1e-4) + np.float32(1e-4) * np.abs(r)).any()
    return {"max_absolute": float(err.max()) if err.size else 0.0, "correct": bool(ok)}


# ---------------------------------------------------------------------------
# Reference dispatch policy and bench constants
# ---------------------------------------------------------------------------
WMMA_M = WMMA_N = WMMA_K = 16

# gemm_bench.cu:45-57 (label, M, N, K)
DEFAULT_SHAPES = [
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


def supports_wmma(m: int, n: int, k: int) -> bool:
    """gemm_bench.cu:252-256."""
    return m % WMMA_M == 0 and n % WMMA_N == 0 and k % WMMA_K == 0


def choose_path_reference(m: int, n: int, k: int, dtype: str) -> str:
    """gemm_bench.cu:260-273: the reference's RTX 3060 dispatch policy."""
    if not supports_wmma(m, n, k):
        return "cublas"
    if dtype == "bf16" and m == 16 and k == 1024 and n >= 4096:
        return "wmma_direct"
    return "cublas"


def repeats_for(flops: float, repeat_override: int = -1) -> int:
    """gemm_bench.cu:371-377: clamp(2e10 / flops, 10, 200)."""
    if repeat_override > 0:
        return repeat_override
    return int(min(max(int(2.0e10 / max(flops, 1.0)), 10), 200))


# ---------------------------------------------------------------------------
# Fused gate/up projection and SiLU-and-mul
# ---------------------------------------------------------------------------
# The Qwen3.5 MLP computes down(SiluAndMul(gate_up(x))) (models/qwen3_5.py:105-118):
# gate_up is a MergedColumnParallelLinear whose W is [W_gate; W_up]
# (layers/linear.py:76-97) and SiluAndMul splits the output in two halves and
# returns F.silu(x) * y (layers/activation.py:8-11).

# max over x of |d/dx (x * sigmoid(x))|; the derivative peaks at 1.0998 near
# x = 2.40 (and is bounded below by -0.0998), so 1.1 bounds |silu'|.
SILU_SLOPE_BOUND = 1.1


def silu_f64(x: np.ndarray) -> np.ndarray:
    """x * sigmoid(x) = x / (1 + exp(-x)) in float64 (exp overflows to inf
    for x < -709, where the quotient is -0 as it should be)."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        return x / (1.0 + np.exp(-x))


def silu_mul_f64(a64: np.ndarray, w64: np.ndarray):
    """SiluAndMul(a @ W^T) for W = [W_gate; W_up] of shape [2n, K]: returns
    (r, g, u) with g = a W_gate^T, u = a W_up^T and r = silu(g) * u, all
    float64."""
    w64 = np.asarray(w64, dtype=np.float64)
    n = w64.shape[0] // 2
    if w64.shape[0] != 2 * n:
        raise ValueError("W must hold gate and up halves of equal height")
    g = gemm_f64(a64, w64[:n])
    u = gemm_f64(a64, w64[n:])
    return silu_f64(g) * u, g, u


def silu_mul_tolerance(r64, g64, u64, sg64, su64, k: int, dtype: str, ulps: float = 2.0) -> np.ndarray:
    """Per-element bound for silu(g~) * u~ evaluated in fp32 from fp32
    accumulations g~, u~ and rounded once to `dtype`.  With dg, du the fp32
    accumulation bounds of g and u (sg, su their sums of |a w|), the mean
    value theorem gives |silu(g~) u~ - silu(g) u| <= 1.1 dg (|u| + du) +
    |silu(g)| du; the fp32 exp, divide and multiply add at most 16 * 2^-24
    of the value; the output rounding is covered by `ulps` units in the last
    place of `dtype` at the exact value."""
    dg = fp32_accumulation_bound(sg64, k)
    du = fp32_accumulation_bound(su64, k)
    return silu_mul_bound(r64, g64, u64, dg, du, dtype, ulps)


def silu_mul_bound(r64, g64, u64, dg, du, dtype: str, ulps: float = 2.0) -> np.ndarray:
    """silu_mul_tolerance for given error bounds dg, du of the two sums."""
    g64 = np.asarray(g64, dtype=np.float64)
    u64 = np.asarray(u64, dtype=np.float64)
    r64 = np.asarray(r64, dtype=np.float64)
    prop = SILU_SLOPE_BOUND * dg * (np.abs(u64) + du) + np.abs(silu_f64(g64)) * du
    evaluation = 16 * 2.0 ** -24 * (np.abs(r64) + prop)
    return ulps * ulp_at(r64, dtype) + prop + evaluation


# ---------------------------------------------------------------------------
# Greedy token of the LM head
# ---------------------------------------------------------------------------
def greedy_tokens(logits: np.ndarray) -> np.ndarray:
    """Greedy rows of Sampler.forward (layers/sampler.py:8-21): argmax of
    the fp32 logits along the vocabulary, first index on ties (torch.argmax)."""
    return np.argmax(np.asarray(logits), axis=-1)


def greedy_token_admissible(token: np.ndarray, r64: np.ndarray, s64: np.ndarray, k: int) -> np.ndarray:
    """True where `token` is a correct greedy choice for logits computed in
    fp32: its exact logit is within twice the fp32 accumulation bound of
    the exact maximum (two logits closer than their error bounds may
    legitimately swap order)."""
    r64 = np.asarray(r64, dtype=np.float64)
    bound = fp32_accumulation_bound(s64, k)
    rows = np.arange(r64.shape[0])
    best = r64.max(axis=-1)
    chosen = r64[rows, token]
    return chosen >= best - bound[rows, token] - bound.max(axis=-1)


def rounded_logit_bounds(r64: np.ndarray, s64: np.ndarray, k: int, dtype: str):
    """(lo, hi) in float64: the smallest and largest value a logit can take
    once an fp32 sum within the accumulation bound of its exact value r is
    rounded to nearest even in `dtype` ("bf16", "f16"), as the reference's
    F.linear in the model dtype does (nanovllm/layers/embed_head.py:61).
    Rounding is monotone, so the ends of [r - b, r + b] bound it."""
    r64 = np.asarray(r64, dtype=np.float64)
    b = fp32_accumulation_bound(s64, k)
    return to_f64(round_f64(r64 - b, dtype), dtype), to_f64(round_f64(r64 + b, dtype), dtype)


def first_argmax_candidates(lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    """mask[i, j]: column j is the first-index argmax of row i for some
    choice of every logit l within [lo, hi] (torch.argmax's rule on the
    reference's logits): l_j can exceed every earlier column's lowest value
    and reach every later column's lowest value, i.e.
    hi_j > max_{c < j} lo_c and hi_j >= max_{c > j} lo_c."""
    lo = np.asarray(lo, dtype=np.float64)
    hi = np.asarray(hi, dtype=np.float64)
    pad = np.full(lo.shape[:-1] + (1,), -np.inf)
    before = np.concatenate([pad, np.maximum.accumulate(lo, axis=-1)[..., :-1]], axis=-1)
    after = np.concatenate([np.maximum.accumulate(lo[..., ::-1], axis=-1)[..., ::-1][..., 1:], pad], axis=-1)
    return (hi > before) & (hi >= after)


def rounded_greedy_candidates(r64: np.ndarray, s64: np.ndarray, k: int, dtype: str) -> np.ndarray:
    """Tokens the reference's greedy rule (argmax of the logits rounded to
    `dtype`, first index on ties; sampler.py:15, 21) can return when each
    logit is summed in fp32 in some order.  A row with a single candidate
    has one right answer whatever the summation order; a row with more
    straddles a rounding boundary within the accumulation bound."""
    lo, hi = rounded_logit_bounds(r64, s64, k, dtype)
    return first_argmax_candidates(lo, hi)


# ---------------------------------------------------------------------------
# Sampled rows of the LM head (Sampler.forward, layers/sampler.py:8-21)
# ---------------------------------------------------------------------------
_PHILOX_MUL = (0xD2511F53, 0xCD9E8D57)
_PHILOX_WEYL = (0x9E3779B9, 0xBB67AE85)
_MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(counters: np.ndarray, key: tuple[int, int]) -> np.ndarray:
    """Philox4x32-10 (Salmon, Moraes, Dror and Shaw, SC 2011) of uint32
    counters [..., 4] under a 2-word key: ten rounds of
    (c0, c1, c2, c3) -> (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0)),
    the key advanced by the Weyl constants between rounds."""
    c = np.asarray(counters, dtype=np.uint64) & _MASK32
    c0, c1, c2, c3 = (c[..., i].copy() for i in range(4))
    k0, k1 = int(key[0]) & 0xFFFFFFFF, int(key[1]) & 0xFFFFFFFF
    for _ in range(10):
        p0 = np.uint64(_PHILOX_MUL[0]) * c0
        p1 = np.uint64(_PHILOX_MUL[1]) * c2
        c0, c1, c2, c3 = ((p1 >> np.uint64(32)) ^ c1 ^ np.uint64(k0), p1 & _MASK32,
                          (p0 >> np.uint64(32)) ^ c3 ^ np.uint64(k1), p0 & _MASK32)
        k0 = (k0 + _PHILOX_WEYL[0]) & 0xFFFFFFFF
        k1 = (k1 + _PHILOX_WEYL[1]) & 0xFFFFFFFF
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def sample_uniform(m: int, n: int, seed: int, offset: int) -> np.ndarray:
    """u[i, j] in (0, 1] of the library's sampled head: the 24 high bits of
    word j % 4 of Philox4x32-10(counter = (j // 4, i, offset, offset >> 32),
    key = (seed, seed >> 32)), plus one, over 2^24 (exact in float64)."""
    rows = np.arange(m, dtype=np.uint64)[:, None]
    cols = np.arange(n, dtype=np.uint64)[None, :]
    ctr = np.empty((m, n, 4), dtype=np.uint64)
    ctr[..., 0] = cols >> np.uint64(2)
    ctr[..., 1] = rows
    ctr[..., 2] = np.uint64(offset & 0xFFFFFFFF)
    ctr[..., 3] = np.uint64((offset >> 32) & 0xFFFFFFFF)
    words = philox4x32_10(ctr, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF))
    word = np.broadcast_to((cols & np.uint64(3)).astype(np.int64)[..., None], (m, n, 1))
    x = np.take_along_axis(words, word, axis=-1)[..., 0]
    return ((x.astype(np.float64) // 256.0) + 1.0) / 2.0 ** 24


def sample_exponential(u: np.ndarray) -> np.ndarray:
    """E = -ln u clamped to >= 1e-10, as the reference clamps its Exp(1)
    draws (sampler.py:20)."""
    return np.maximum(-np.log(np.asarray(u, dtype=np.float64)), 1e-10)


def sample_scores_f64(logits: np.ndarray, temperatures: np.ndarray, e: np.ndarray) -> np.ndarray:
    """Rank of every column: the logit on a greedy row (temperature <= 1e-10
    in float32, sampler.py:9), l / T - ln E on a sampled one (the Gumbel-max
    form of the reference's softmax(l / T) / E)."""
    logits = np.asarray(logits, dtype=np.float64)
    t = np.asarray(temperatures, dtype=np.float32)
    greedy = (t <= np.float32(1e-10))[:, None]
    safe_t = np.where(greedy[:, 0], 1.0, t.astype(np.float64))[:, None]
    return np.where(greedy, logits, logits / safe_t - np.log(e))


def sampler_reference_f64(logits: np.ndarray, temperatures: np.ndarray, e: np.ndarray) -> np.ndarray:
    """Sampler.forward (sampler.py:9-21) restated in float64 for given noise
    E: greedy rows take argmax l; the others argmax softmax(l / T) / E."""
    logits = np.asarray(logits, dtype=np.float64)
    t = np.asarray(temperatures, dtype=np.float32)
    greedy = t <= np.float32(1e-10)
    safe_t = np.where(greedy, 1.0, t.astype(np.float64))[:, None]
    z = logits / safe_t
    p = np.exp(z - z.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    sample = (p / e).argmax(axis=-1)
    return np.where(greedy, logits.argmax(axis=-1), sample)


def sample_token_admissible(token: np.ndarray, r64: np.ndarray, s64: np.ndarray, k: int,
                            temperatures: np.ndarray, e: np.ndarray, logit_dtype: str = "f32") -> np.ndarray:
    """True where `token` is a correct choice of the sampled head for fp32
    logits: its exact score is within the error budget of the best exact
    score.  The budget is the fp32 accumulation bound of each logit over T
    (twice, as two logits may swap), plus 4e-6 (1 + |score|) for the fp32
    division, the hardware logarithms and the draw's fp32 E.

    logit_dtype "bf16" / "f16": the logits are rounded to that type first
    (the reference's model-dtype logits); every logit then lies in
    rounded_logit_bounds, and the token's highest possible score must reach
    the best lowest possible score of the row."""
    t = np.asarray(temperatures, dtype=np.float32)
    greedy = t <= np.float32(1e-10)
    if logit_dtype != "f32":
        lo, hi = rounded_logit_bounds(r64, s64, k, logit_dtype)
        sc_lo = sample_scores_f64(lo, temperatures, e)
        sc_hi = sample_scores_f64(hi, temperatures, e)
        slack = np.where(greedy[:, None], 0.0, 4e-6 * (1.0 + np.abs(sc_hi)))
        rows = np.arange(sc_hi.shape[0])
        return sc_hi[rows, token] + slack[rows, token] >= (sc_lo - slack).max(axis=-1)
    scale = np.where(greedy, 1.0, 1.0 / np.where(greedy, 1.0, t.astype(np.float64)))[:, None]
    sc = sample_scores_f64(r64, temperatures, e)
    bound = fp32_accumulation_bound(s64, k) * scale + np.where(greedy[:, None], 0.0, 4e-6 * (1.0 + np.abs(sc)))
    rows = np.arange(sc.shape[0])
    best = sc.max(axis=-1)
    chosen = sc[rows, token]
    return chosen >= best - bound[rows, token] - bound.max(axis=-1)


# ---------------------------------------------------------------------------
# Prologues on A
# ---------------------------------------------------------------------------
def sigmoid_f64(x: np.ndarray) -> np.ndarray:
    """1 / (1 + e^-x) in float64."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-x))


def gate_view(gate_rows: np.ndarray, k: int, group: int, group_stride: int) -> np.ndarray:
    """The [m, k] gate read through q_proj's head-strided view
    (nanovllm/models/qwen3_5.py:81-86): element (i, k) is
    gate_rows[i, (k // group) * group_stride + k % group], where row i of
    gate_rows starts at the gate's first element (for the chunk of q_proj's
    output, head_dim elements into the row)."""
    j = np.arange(k)
    return np.asarray(gate_rows)[:, (j // group) * group_stride + j % group]


def sigmoid_gate(a: np.ndarray, g: np.ndarray, dtype: str) -> np.ndarray:
    """The output gate of gated attention, `output * torch.sigmoid(gate)`
    (qwen3_5.py:95), as two element-type tensor ops: sigmoid(g) rounded to
    `dtype`, then the product (exact in float64 for bf16 and fp16 factors)
    rounded to `dtype`.  a and g are storage arrays of `dtype`."""
    s = to_f64(round_f64(sigmoid_f64(to_f64(g, dtype)), dtype), dtype)
    return round_f64(to_f64(a, dtype) * s, dtype)


def add_norm_operand(h: np.ndarray, r: np.ndarray, w_norm: np.ndarray, dtype: str):
    """Residual add + zero-centred RMSNorm operand as the kernels form it
    (Qwen3_5RMSNorm with a residual, nanovllm/layers/layernorm.py:131-142,
    with the row scale moved behind the GEMM): s = h + r in fp32, the new
    residual round(s) (as the reference), the GEMM operand
    round(fp32(s * fp32(1 + w))).  Each fp32 operation is its float64 value
    (exact for these factors) rounded once.  Returns (s as float64, operand
    storage, residual storage)."""
    s32 = (to_f64(h, dtype) + to_f64(r, dtype)).astype(np.float32)
    one_w = (1.0 + to_f64(w_norm, dtype)).astype(np.float32)
    y32 = (s32.astype(np.float64) * one_w.astype(np.float64)).astype(np.float32)
    return s32.astype(np.float64), encode(y32, dtype), encode(s32, dtype)


def norm_scale_f64(s64: np.ndarray, eps: float) -> np.ndarray:
    """rsqrt(mean_k s^2 + eps) per row, in float64 (layernorm.py:126-128)."""
    s64 = np.asarray(s64, dtype=np.float64)
    return 1.0 / np.sqrt((s64 * s64).mean(axis=-1) + eps)


def norm_scale_error(k: int) -> float:
    """Relative error bound of the fp32 row scale: the sum of k positive
    squares (k 2^-24), the divide by k and the add of eps, the square root
    (which halves the error of its input) and the reciprocal, plus the
    multiply that applies it: (k / 2 + 4) 2^-24, taken as k 2^-24 + 2^-21."""
    return k * 2.0 ** -24 + 2.0 ** -21


def add_norm_gemm_tolerance(r64, sy64, scale64, k: int, dtype: str, ulps: float = 2.0) -> np.ndarray:
    """Bound for scale~ * (fp32 sum of the operand times w) rounded once to
    `dtype`, against r64 = scale * sum in float64: the fp32 accumulation
    (scaled), the fp32 row scale's relative error on the value, `ulps` of
    the output type.  sy64 = sum_k |y w|."""
    r64 = np.asarray(r64, dtype=np.float64)
    scale = np.asarray(scale64, dtype=np.float64)[:, None]
    return (ulps * ulp_at(r64, dtype) + scale * fp32_accumulation_bound(sy64, k)
            + norm_scale_error(k) * np.abs(r64))
