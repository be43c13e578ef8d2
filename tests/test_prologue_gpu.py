"""GPU parity of the GEMMs with a prologue on A: the output gate of gated
attention in front of o_proj (nanovllm/models/qwen3_5.py:95-96) and the
residual add + zero-centred RMSNorm in front of a projection
(nanovllm/layers/layernorm.py:131-142), fused into splitk_decode for M <= 32
and run as a prologue kernel + GEMM above.

Bars:
  * the standalone gate kernel against the oracle's two-rounding gate
    (sigmoid rounded to the element type, then the product): within 1 ulp
    everywhere and bit-exact for >= 99.9% of the elements (fp32 sigmoid and
    the float64 one round differently only next to a rounding tie);
  * the fused gated GEMM bit-exact against the gate kernel followed by the
    plain GEMM on the same kernel (same operand bits, same sum order), and
    that against the oracle's GEMM bound;
  * add + RMSNorm: the new residual bit-exact against round(h + r); the
    output against the oracle's float64 evaluation of the kernels' formula
    (operand round(s (1 + w)), row scale rsqrt(mean s^2 + eps) applied to
    the sum) with the fp32 accumulation and row-scale error bounds plus 2
    ulp of the output type.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import PKG
from oracle import gemm_oracle as orc

pytestmark = pytest.mark.gpu

L = PKG._lib
K = PKG.kernels
DEV = torch.device("cuda:0")
NAME = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def _say(msg):
    print(msg, flush=True)


def _store(t: torch.Tensor) -> np.ndarray:
    """Tensor -> oracle storage (bf16 as uint16 bits)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def _value(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().double().numpy()


def _qgate(m, heads, head_dim, dtype, gen):
    """q_proj output viewed as (M, heads, 2 head_dim) and its gate half (qwen3_5.py:81-86)."""
    q_gate = (torch.randn((m, heads, 2 * head_dim), generator=gen) * 3).to(dtype)
    return q_gate, q_gate.chunk(2, dim=-1)[1]


# ---------------------------------------------------------------------------
# Output gate
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("view", ["heads", "contiguous"])
def test_sigmoid_gate_kernel_vs_oracle(dtype, view):
    gen = torch.Generator().manual_seed(7)
    m, heads, hd = 37, 8, 256
    a = torch.randn((m, heads, hd), generator=gen).to(dtype)
    q_gate, gate = _qgate(m, heads, hd, dtype, gen)
    if view == "contiguous":
        gate = gate.contiguous().view(m, heads * hd)
    _say(f"sigmoid_gate {NAME[dtype]} {view} M={m}")
    got = K.sigmoid_gate(a.to(DEV), gate.to(DEV) if view == "contiguous" else q_gate.to(DEV).chunk(2, -1)[1])
    torch.cuda.synchronize()
    k = heads * hd
    g_rows = _store(q_gate.view(m, -1))[:, hd:]      # rows from the gate's first element
    g_store = orc.gate_view(g_rows, k, hd, 2 * hd)
    want = orc.sigmoid_gate(_store(a.view(m, k)), g_store, NAME[dtype])
    ulps = orc.ulp_distance(_store(got), want, NAME[dtype])
    assert ulps.max() <= 1, int(ulps.max())
    assert float((ulps == 0).mean()) >= 0.999
    # and torch's own composition on the GPU (the reference's two ops)
    ref = (a.to(DEV) * torch.sigmoid(q_gate.to(DEV).chunk(2, -1)[1])).view(m, k)
    assert float((ref == got).float().mean()) >= 0.999


@pytest.mark.parametrize("m", [1, 5, 16, 32])
@pytest.mark.parametrize("n", [1024, 9000])
@pytest.mark.parametrize("dtype,dout", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)],
                         ids=["bf16", "f16-f32"])
def test_gemm_gated_fused_equals_gate_then_gemm(m, n, dtype, dout):
    """Qwen3.5 o_proj (N = 1024, K = 8 heads x 256), and a W wide enough
    (9000 rows) for the wide-W configurations: the gate inside splitk_decode
    (forced here at every M; the default fuses it up to M = 8) gives the same
    bits as the gate kernel followed by splitk_decode, and so does the
    default path; that meets the GEMM bound on the gated operand."""
    gen = torch.Generator().manual_seed(100 + m + n)
    heads, hd = 8, 256
    a = torch.randn((m, heads, hd), generator=gen).to(dtype).to(DEV)
    q_gate, _ = _qgate(m, heads, hd, dtype, gen)
    gate = q_gate.to(DEV).chunk(2, -1)[1]
    w = (torch.randn((n, heads * hd), generator=gen) * 0.02).to(dtype).to(DEV)
    _say(f"gemm_gated fused M={m} N={n} {NAME[dtype]}->{NAME[dout]}")
    fused = K.gemm_gated_with_kernel(a, gate, w, L.KERNEL_SPLITK_DECODE, dout)
    default = K.gemm_gated(a, gate, w, dout)
    operand = K.sigmoid_gate(a, gate)
    composed = PKG.kernels.gemm_with_kernel(operand, w, L.KERNEL_SPLITK_DECODE, dout)
    torch.cuda.synchronize()
    assert torch.equal(fused, composed)
    assert torch.equal(default, composed)
    a64, w64 = _value(operand), _value(w)
    r = orc.gemm_f64(a64, w64)
    tol = orc.gemm_tolerance(r, orc.abs_products_f64(a64, w64), heads * hd, NAME[dout])
    err = np.abs(_value(fused) - r)
    assert (err <= tol).all(), float((err - tol).max())


@pytest.mark.parametrize("m,hd", [(300, 256), (4, 40), (40, 128)], ids=["staged", "group40", "m40"])
def test_gemm_gated_prologue_kernel_path(m, hd):
    """Problems the fused gate does not take (M > 32, or a head_dim that is
    not a multiple of 64) run the gate kernel into the workspace and then the
    GEMM the table selects: bit-exact against sigmoid_gate + gemm."""
    gen = torch.Generator().manual_seed(m + hd)
    heads, n = 4, 520
    a = torch.randn((m, heads, hd), generator=gen).bfloat16().to(DEV)
    q_gate, _ = _qgate(m, heads, hd, torch.bfloat16, gen)
    gate = q_gate.to(DEV).chunk(2, -1)[1]
    w = (torch.randn((n, heads * hd), generator=gen) * 0.05).bfloat16().to(DEV)
    _say(f"gemm_gated prologue path M={m} head_dim={hd}")
    got = K.gemm_gated(a, gate, w)
    want = PKG.kernels.gemm(K.sigmoid_gate(a, gate), w)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_gemm_gated_contract_errors_on_gpu():
    a = torch.randn(4, 2, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.randn(32, 128, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(4, 2, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="gate shape"):
        K.gemm_gated(a, torch.randn(4, 3, 64, device=DEV, dtype=torch.bfloat16), w)
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        K.gemm_gated(a.float(), q.float().chunk(2, -1)[1], w.float())
    with pytest.raises(RuntimeError, match="unit stride"):
        K.gemm_gated(a, q[:, :, ::2], w)


# ---------------------------------------------------------------------------
# Residual add + RMSNorm
# ---------------------------------------------------------------------------
def _norm_inputs(m, n_rows, k, dtype, gen, tiny_row=True):
    h = torch.randn((m, k), generator=gen).to(dtype)
    r = torch.randn((m, k), generator=gen).to(dtype)
    if tiny_row and m > 1:
        # a row whose mean square is of the order of eps
        h[1] = (torch.randn(k, generator=gen) * 1e-3).to(dtype)
        r[1] = (torch.randn(k, generator=gen) * 1e-3).to(dtype)
    nw = (torch.randn(k, generator=gen) * 0.1).to(dtype)
    w = (torch.randn((n_rows, k), generator=gen) * 0.05).to(dtype)
    return h, r, nw, w


def _norm_oracle(h, r, nw, w, eps, dtype):
    s64, y, res = orc.add_norm_operand(_store(h), _store(r), _store(nw), NAME[dtype])
    scale = orc.norm_scale_f64(s64, eps)
    y64 = orc.to_f64(y, NAME[dtype])
    return y64, scale, res


def _check_add_norm(out, res_out, h, r, nw, w, eps, dtype, dout):
    """The new residual bit-exact; the output within the oracle's bound of
    scale * (y w^T) in float64 and, for narrow outputs, every element within
    2 ulp of the fp32 reference (host fp32 GEMM of the same operand y, times
    the fp32 row scale, rounded once) but a few cancellation elements
    (oracle.narrow_parity)."""
    y64, scale, res = _norm_oracle(h, r, nw, w, eps, dtype)
    assert np.array_equal(_store(res_out), res), "new residual differs from round(h + r)"
    w64 = _value(w)
    k = h.shape[1]
    r64 = scale[:, None] * orc.gemm_f64(y64, w64)
    tol = orc.add_norm_gemm_tolerance(r64, orc.abs_products_f64(y64, w64), scale, k, NAME[dout])
    got = _value(out)
    assert np.isfinite(got).all()
    err = np.abs(got - r64)
    assert (err <= tol).all(), f"{int((err > tol).sum())} outside; worst excess {float((err - tol).max()):.3g}"
    if dout != torch.float32:
        y32 = torch.from_numpy(y64.astype(np.float32))
        scale32 = torch.from_numpy(scale.astype(np.float32))
        ref32 = (y32 @ torch.from_numpy(w64.astype(np.float32)).T) * scale32[:, None]
        ref = _store(ref32.to(dout))
        stats = orc.narrow_parity(_store(out), ref, r64, scale[:, None] * orc.abs_products_f64(y64, w64), NAME[dout])
        ok = stats.pop("ok")
        print(f"  narrow {NAME[dout]}: {ok.size} outputs, {stats['cancel_beyond']} cancellation elements beyond 2 ulp "
              f"(cap {orc.cancellation_cap(ok.size, NAME[dout])}), max ulp {stats['max_ulp_checked']}", flush=True)
        assert ok.all(), f"{int((~ok).sum())} elements beyond 2 ulp of the fp32 reference ({stats})"
        assert stats["cancel_beyond"] <= orc.cancellation_cap(ok.size, NAME[dout]), stats


NORM_SHAPES = [(6144, 1024), (1000, 1000), (1024, 3584), (3000, 3592), (9000, 1000)]


@pytest.mark.parametrize("n,k", NORM_SHAPES, ids=[f"N{n}-K{k}" for n, k in NORM_SHAPES])
@pytest.mark.parametrize("m", [1, 7, 16, 32])
@pytest.mark.parametrize("dtype,dout", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32)],
                         ids=["bf16", "bf16-f32"])
def test_add_rmsnorm_fused(n, k, m, dtype, dout):
    gen = torch.Generator().manual_seed(n + k + m)
    h, r, nw, w = _norm_inputs(m, n, k, dtype, gen)
    eps = 1e-6
    _say(f"add_rmsnorm fused M={m} N={n} K={k} {NAME[dtype]}->{NAME[dout]}")
    out, res_out = K.gemm_add_rmsnorm(h.to(DEV), r.to(DEV), nw.to(DEV), w.to(DEV), eps, out_dtype=dout)
    torch.cuda.synchronize()
    _check_add_norm(out, res_out, h, r, nw, w, eps, dtype, dout)


def _check_add_norm_silu(out, res_out, h, r, nw, w, eps, dtype, dout):
    y64, scale, res = _norm_oracle(h, r, nw, w, eps, dtype)
    assert np.array_equal(_store(res_out), res)
    k = h.shape[1]
    n = w.shape[0] // 2
    w64 = _value(w)
    g = scale[:, None] * orc.gemm_f64(y64, w64[:n])
    u = scale[:, None] * orc.gemm_f64(y64, w64[n:])
    r64 = orc.silu_f64(g) * u
    eps_r = orc.norm_scale_error(k)
    dg = scale[:, None] * orc.fp32_accumulation_bound(orc.abs_products_f64(y64, w64[:n]), k) + eps_r * np.abs(g)
    du = scale[:, None] * orc.fp32_accumulation_bound(orc.abs_products_f64(y64, w64[n:]), k) + eps_r * np.abs(u)
    tol = orc.silu_mul_bound(r64, g, u, dg, du, NAME[dout])
    err = np.abs(_value(out) - r64)
    assert (err <= tol).all(), f"{int((err > tol).sum())} outside; worst excess {float((err - tol).max()):.3g}"


@pytest.mark.parametrize("m,n,k", [(1, 3584, 1024), (4, 3584, 1024), (32, 3584, 1024), (9, 500, 136)],
                         ids=["qwen-M1", "qwen-M4", "qwen-M32", "ragged"])
def test_add_rmsnorm_silu_fused(m, n, k):
    """Add + RMSNorm + gate_up + SiluAndMul in one splitk_decode launch (the
    Qwen3.5-0.8B MLP block at decode: 2 x 3584 rows, K = 1024)."""
    gen = torch.Generator().manual_seed(m * 3 + n)
    h, r, nw, w = _norm_inputs(m, 2 * n, k, torch.bfloat16, gen)
    _say(f"add_rmsnorm silu fused M={m} N={n} K={k}")
    out, res_out = K.gemm_add_rmsnorm(h.to(DEV), r.to(DEV), nw.to(DEV), w.to(DEV), 1e-6, silu_mul=True)
    torch.cuda.synchronize()
    assert out.shape == (m, n)
    _check_add_norm_silu(out, res_out, h, r, nw, w, 1e-6, torch.bfloat16, torch.bfloat16)


@pytest.mark.parametrize("m,silu", [(300, False), (100, True), (20, False)], ids=["M300", "M100-silu", "M20-forced"])
def test_add_rmsnorm_prologue_kernel_path(m, silu):
    """Above M = 32 (or forced onto mfma_staged) the prologue kernel writes
    the operand and the row scales to the workspace and mfma_staged scales
    its output rows."""
    gen = torch.Generator().manual_seed(m)
    k, n = 1000, 700
    h, r, nw, w = _norm_inputs(m, 2 * n if silu else n, k, torch.bfloat16, gen)
    args = (h.to(DEV), r.to(DEV), nw.to(DEV), w.to(DEV), 1e-5)
    _say(f"add_rmsnorm prologue path M={m} silu={silu}")
    if m <= 32:
        out, res_out = K.gemm_add_rmsnorm_with_kernel(*args, L.KERNEL_MFMA_STAGED, silu_mul=silu)
    else:
        out, res_out = K.gemm_add_rmsnorm(*args, silu_mul=silu)
    torch.cuda.synchronize()
    if silu:
        _check_add_norm_silu(out, res_out, h, r, nw, w, 1e-5, torch.bfloat16, torch.bfloat16)
    else:
        _check_add_norm(out, res_out, h, r, nw, w, 1e-5, torch.bfloat16, torch.bfloat16)


@pytest.mark.parametrize("m,n,silu", [(1500, 2000, False), (2100, 2000, False), (2100, 1000, True),
                                      (2100, 4100, False)],
                         ids=["128x128-spread", "128x256", "128x256-silu", "128x128-2deep"])
def test_add_rmsnorm_row_scale_large_grids(m, n, silu):
    """The row-scaled epilogue on mfma_staged's large-grid tiles: 192 tiles
    of 128 x 128 (3-deep ring, spread copies), 136 tiles of 128 x 256 (8
    waves, spread copies; plain and with SiLU-and-mul) and 289 (where 128 x
    128 with a 2-deep ring takes over); ragged M, N and K."""
    gen = torch.Generator().manual_seed(m + n)
    k = 1000
    h, r, nw, w = _norm_inputs(m, 2 * n if silu else n, k, torch.bfloat16, gen)
    _say(f"add_rmsnorm large grid M={m} N={n} silu={silu}")
    out, res_out = K.gemm_add_rmsnorm(h.to(DEV), r.to(DEV), nw.to(DEV), w.to(DEV), 1e-5, silu_mul=silu)
    torch.cuda.synchronize()
    if silu:
        _check_add_norm_silu(out, res_out, h, r, nw, w, 1e-5, torch.bfloat16, torch.bfloat16)
    else:
        _check_add_norm(out, res_out, h, r, nw, w, 1e-5, torch.bfloat16, torch.bfloat16)


def test_add_rmsnorm_close_to_reference_composition():
    """The reassociated row scale stays close to Qwen3_5RMSNorm + F.linear
    computed by torch on the GPU, which rounds the normalized activations
    before the GEMM where the fused path rounds s (1 + w) and scales the
    sum: the same new residual; the two roundings of ~1024 terms move an
    output by a fraction of an ulp each way (measured: 89% of the outputs
    within 2 bf16 ulp, the rest where outputs cancel toward zero), and the
    relative Frobenius distance stays at the bf16 rounding level."""
    gen = torch.Generator().manual_seed(3)
    h, r, nw, w = _norm_inputs(8, 6144, 1024, torch.bfloat16, gen, tiny_row=False)
    hd, rd, nwd, wd = h.to(DEV), r.to(DEV), nw.to(DEV), w.to(DEV)
    out, res_out = K.gemm_add_rmsnorm(hd, rd, nwd, wd, 1e-6)
    ref, ref_res = K.add_rmsnorm_linear(hd, rd, nwd, 1e-6, wd, backend="torch")
    torch.cuda.synchronize()
    assert torch.equal(res_out, ref_res)
    ulps = orc.ulp_distance(_store(out), _store(ref), "bf16")
    assert float((ulps <= 2).mean()) >= 0.85
    assert orc.rel_frobenius(_value(out), _value(ref)) <= 5e-3


def test_prologue_ops_graph_capture():
    """Both fused ops (and the workspace path) captured in one HIP graph and
    replayed, each replay equal to the eager result."""
    gen = torch.Generator().manual_seed(5)
    h, r, nw, w = (t.to(DEV) for t in _norm_inputs(4, 3000, 1024, torch.bfloat16, gen))
    h64, r64, nw64, w64 = (t.to(DEV) for t in _norm_inputs(64, 3000, 1024, torch.bfloat16, gen))
    a = torch.randn((4, 8, 256), generator=gen).bfloat16().to(DEV)
    q = torch.randn((4, 8, 512), generator=gen).bfloat16().to(DEV)
    wo = (torch.randn((1024, 2048), generator=gen) * 0.02).bfloat16().to(DEV)

    def step():
        return (K.gemm_add_rmsnorm(h, r, nw, w, 1e-6), K.gemm_add_rmsnorm(h64, r64, nw64, w64, 1e-6),
                K.gemm_gated(a, q.chunk(2, -1)[1], wo))

    eager = step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        static = step()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        _ = step()   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(static[0][0], eager[0][0]) and torch.equal(static[0][1], eager[0][1]), rep
        assert torch.equal(static[1][0], eager[1][0]) and torch.equal(static[1][1], eager[1][1]), rep
        assert torch.equal(static[2], eager[2]), rep
