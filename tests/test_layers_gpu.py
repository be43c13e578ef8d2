"""GPU tests of the layer mirrors on the HIP path (backend "hip").

The decode loop of the reference replays its forward inside a CUDA graph
(nanovllm/engine/model_runner.py:1795-1911), so a Qwen3.5-0.8B-shaped MLP
block (gate_up N = 2 x 3584, SiLU-and-mul, down K = 3584;
nanovllm/models/qwen3_5.py:105-118) is captured in a HIP graph here and every
replay is compared with eager execution, bit for bit (the kernels are
deterministic)."""
from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import PKG
from oracle import gemm_oracle as orc

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
Lyr = PKG.layers
G = importlib.import_module("inference_systems_amd.kernels.gemm")


def _init(layer, gen, scale=0.02):
    with torch.no_grad():
        layer.weight.copy_(torch.randn(layer.weight.shape, generator=gen) * scale)
        if getattr(layer, "bias", None) is not None:
            layer.bias.copy_(torch.randn(layer.bias.shape, generator=gen) * scale)
    return layer


@torch.inference_mode()
def test_layers_hip_match_op():
    gen = torch.Generator().manual_seed(21)
    x = torch.randn(40, 1024, generator=gen).bfloat16().to(DEV)
    for layer in (Lyr.ReplicatedLinear(1024, 768, bias=True), Lyr.ColumnParallelLinear(1024, 512),
                  Lyr.QKVParallelLinear(1024, 128, 16, 8), Lyr.RowParallelLinear(1024, 256, bias=True)):
        layer = _init(layer, gen).to(DEV, torch.bfloat16)
        layer.gemm_backend = "hip"
        y = layer(x)
        ref = G.gemm(x, layer.weight)
        if layer.bias is not None:
            ref = ref + layer.bias
        assert torch.equal(y, ref), type(layer).__name__


@pytest.mark.parametrize("m", [1, 8, 300])
def test_lm_head_fp32_logits(m):
    """The fp32-logit opt-in of the LM head: the GEMM writes fp32 logits
    within the fp32 bound of the float64 product."""
    gen = torch.Generator().manual_seed(22)
    vocab, hidden = 151936, 1024
    head = Lyr.ParallelLMHead(vocab, hidden)
    with torch.no_grad():
        head.weight.copy_(torch.randn(vocab, hidden, generator=gen) * 0.02)
    head = head.to(DEV, torch.bfloat16)
    head.gemm_backend = "hip"
    head.logits_dtype = torch.float32
    x = torch.randn(m + 3, hidden, generator=gen).bfloat16()
    last = torch.arange(m) + 3
    with torch.inference_mode():        # the reference runs its model in inference mode
        logits = head(x.to(DEV), last.to(DEV))
    torch.cuda.synchronize()
    assert logits.dtype == torch.float32 and logits.shape == (m, vocab)
    rows = np.unique(np.linspace(0, m - 1, min(m, 16)).astype(int))
    a64 = x[last].double().numpy()[rows]
    w64 = head.weight.detach().double().cpu().numpy()
    r = orc.gemm_f64(a64, w64)
    tol = orc.gemm_tolerance(r, orc.abs_products_f64(a64, w64), hidden, "f32")
    got = logits.cpu().double().numpy()[rows]
    assert (np.abs(got - r) <= tol).all()


class _QwenMLP(torch.nn.Module):
    """gate_up (merged column) -> SiLU(gate) * up -> down (row parallel)."""

    def __init__(self, hidden=1024, inter=3584):
        super().__init__()
        self.gate_up = Lyr.MergedColumnParallelLinear(hidden, [inter, inter])
        self.down = Lyr.RowParallelLinear(inter, hidden)

    def forward(self, x):
        gu = self.gate_up(x)
        gate, up = gu.chunk(2, -1)
        return self.down((F.silu(gate) * up).contiguous())


@pytest.mark.parametrize("m", [4, 32])
@torch.inference_mode()
def test_mlp_block_graph_capture(m):
    gen = torch.Generator().manual_seed(23)
    mlp = _QwenMLP()
    for layer in (mlp.gate_up, mlp.down):
        _init(layer, gen)
        layer.gemm_backend = "hip"
    mlp = mlp.to(DEV, torch.bfloat16)
    x_static = torch.zeros(m, 1024, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mlp(x_static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_static = mlp(x_static)
    for step in range(3):
        x = torch.randn(m, 1024, generator=gen).bfloat16().to(DEV)
        x_static.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        eager = mlp(x)
        torch.cuda.synchronize()
        assert torch.equal(y_static, eager), f"replay {step}"
    # and the block agrees with the F.linear path within bf16 tolerance
    for layer in (mlp.gate_up, mlp.down):
        layer.gemm_backend = "torch"
    ref = mlp(x).float()
    assert torch.allclose(eager.float(), ref, rtol=0.05, atol=0.02)


@torch.inference_mode()
@pytest.mark.parametrize("m", [1, 4, 32, 48, 300])
def test_gdn_merged_projection_bit_exact(m):
    """Qwen3.5-0.8B gated-delta-net input projections (hidden 1024; 16 key
    and 16 value heads of 128; N = 6144 + 2048 + 16 + 16 = 8224) as one GEMM:
    every kernel's per-element arithmetic is independent of N, so the merged
    launch must equal the four separate launches bit for bit, and the oracle
    bound like any other GEMM."""
    gen = torch.Generator().manual_seed(40 + m)
    proj = Lyr.GdnInputProjection(1024, 16, 16, 128, 128)
    parts = {sid: torch.randn(rows, 1024, generator=gen) * 0.02
             for sid, rows in (("qkv", 6144), ("z", 2048), ("b", 16), ("a", 16))}
    for sid, w in parts.items():
        proj.weight.weight_loader(proj.weight, w, sid)
    proj = proj.to(DEV, torch.bfloat16)
    proj.gemm_backend = "hip"
    x = torch.randn(m, 1024, generator=gen).bfloat16()
    print(f"gdn merged projection M={m}", flush=True)
    merged = proj(x.to(DEV))
    torch.cuda.synchronize()
    for out, sid in zip(merged, ("qkv", "z", "b", "a")):
        w = parts[sid].bfloat16()
        single = G.gemm(x.to(DEV), w.to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(out, single), sid
    # contiguous outputs (four GEMMs on the weight's row ranges) are the same values
    for out, part in zip(merged, proj(x.to(DEV), contiguous=True)):
        assert part.is_contiguous() and torch.equal(out, part)
    got = torch.cat(merged, dim=-1).cpu()
    wall = torch.cat([parts[s].bfloat16() for s in ("qkv", "z", "b", "a")], dim=0)
    a64, w64 = x.double().numpy(), wall.double().numpy()
    r = orc.gemm_f64(a64, w64, "nk")
    tol = orc.gemm_tolerance(r, orc.abs_products_f64(a64, w64, "nk"), 1024, "bf16")
    assert (np.abs(got.double().numpy() - r) <= tol).all()


@pytest.mark.parametrize("m", [1, 32, 256])
@torch.inference_mode()
def test_qwen35_mlp_fused_graph_capture(m):
    """Qwen35MLP on the HIP path (gate_up + SiLU-and-mul fused, then down)
    captured in a HIP graph: every replay equals eager execution bit for bit,
    and the block agrees with the unfused composition within bf16 tolerance."""
    gen = torch.Generator().manual_seed(60 + m)
    mlp = Lyr.Qwen35MLP(1024, 3584)
    _init(mlp.gate_up_proj, gen)
    _init(mlp.down_proj, gen)
    mlp = mlp.to(DEV, torch.bfloat16)
    mlp.gemm_backend = "hip"
    x_static = torch.zeros(m, 1024, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mlp(x_static)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_static = mlp(x_static)
    for step in range(3):
        x = torch.randn(m, 1024, generator=gen).bfloat16().to(DEV)
        x_static.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        eager = mlp(x)
        torch.cuda.synchronize()
        assert torch.equal(y_static, eager), f"replay {step}"
    mlp.gemm_backend = "torch"
    ref = mlp(x).float()
    assert torch.allclose(eager.float(), ref, rtol=0.05, atol=0.02)


@torch.inference_mode()
@pytest.mark.parametrize("m", [1, 8, 32])
def test_lm_head_greedy_hip(m):
    """ParallelLMHead.greedy on the HIP path equals the argmax of the head's
    own logits (bf16 by default, as the reference's F.linear returns them;
    fp32 when opted in), from the same kernel configuration for the Qwen3.5
    vocabulary."""
    gen = torch.Generator().manual_seed(80 + m)
    head = _init(Lyr.ParallelLMHead(151936, 1024), gen).to(DEV, torch.bfloat16)
    head.gemm_backend = "hip"
    x = torch.randn(m + 3, 1024, generator=gen).bfloat16().to(DEV)
    last = torch.arange(m, device=DEV) + 3
    head.logits_dtype = torch.float32
    t32, v32 = head.greedy(x, last)
    l32 = head(x, last)
    head.logits_dtype = None
    tokens, values = head.greedy(x, last)
    logits = head(x, last)
    torch.cuda.synchronize()
    assert logits.dtype == torch.bfloat16 and l32.dtype == torch.float32
    assert torch.equal(t32, l32.argmax(-1)) and torch.equal(v32, l32.gather(-1, t32[:, None]).squeeze(-1))
    logits = logits.float()
    assert torch.equal(tokens, logits.argmax(-1))
    assert torch.equal(values, logits.gather(-1, tokens[:, None]).squeeze(-1))


@torch.inference_mode()
@pytest.mark.parametrize("m", [1, 32, 40])
def test_lm_head_sample_hip(m):
    """ParallelLMHead.sample on the HIP path (Qwen3.5 vocabulary): greedy
    rows equal ParallelLMHead.greedy, sampled rows are admissible draws for
    the oracle's noise (checked on the oracle's float64 logits of the head's
    own bf16 weights, rounded to bf16 as the reference's logits are), and
    the torch backend (the reference Sampler on torch's bf16 logits) returns
    the same greedy token on every row whose token the oracle fixes whatever
    the fp32 summation order (one candidate); on a row whose top logits
    straddle a bf16 rounding boundary within the accumulation bound both
    tokens must be candidates."""
    gen = torch.Generator().manual_seed(90 + m)
    head = _init(Lyr.ParallelLMHead(151936, 1024), gen).to(DEV, torch.bfloat16)
    head.gemm_backend = "hip"
    x = torch.randn(m, 1024, generator=gen).bfloat16().to(DEV)
    temps = torch.rand(m, generator=gen) + 0.5
    temps[::2] = 0.0
    seed, offset = 1234, 56
    tokens, scores = head.sample(x, temps.to(DEV), seed, offset)
    g_tokens, _ = head.greedy(x)
    logits = head(x).cpu()
    head.gemm_backend = "torch"
    t_tokens, t_scores = head.sample(x, temps.to(DEV), seed, offset)
    torch.cuda.synchronize()
    greedy = temps <= 1e-10
    assert t_scores is None
    assert torch.equal(tokens.cpu()[greedy], g_tokens.cpu()[greedy])
    assert ((t_tokens >= 0) & (t_tokens < 151936)).all()
    assert logits.dtype == torch.bfloat16          # the reference's model-dtype logits
    a64 = x.double().cpu().numpy()
    w64 = head.weight.double().cpu().numpy()
    r = orc.gemm_f64(a64, w64)
    s = orc.abs_products_f64(a64, w64)
    cand = orc.rounded_greedy_candidates(r[greedy.numpy()], s[greedy.numpy()], 1024, "bf16")
    ours, theirs = tokens.cpu()[greedy].numpy(), t_tokens.cpu()[greedy].numpy()
    rows = np.arange(len(ours))
    assert cand[rows, ours].all() and cand[rows, theirs].all()
    one = cand.sum(-1) == 1
    np.testing.assert_array_equal(ours[one], theirs[one])
    print(f"greedy rows {len(ours)}: {int(one.sum())} with one candidate, {int((~one).sum())} straddling", flush=True)
    e = orc.sample_exponential(orc.sample_uniform(m, 151936, seed, offset))
    ok = orc.sample_token_admissible(tokens.cpu().numpy(), r, s, 1024, temps.numpy(), e, "bf16")
    assert ok.all()


def _norm(gen, hidden=1024):
    norm = Lyr.Qwen35RMSNorm(hidden)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(hidden, generator=gen) * 0.1)
    return norm.to(DEV, torch.bfloat16)


@pytest.mark.parametrize("m", [1, 8, 32, 100])
@torch.inference_mode()
def test_mlp_forward_add_norm_hip_graph(m):
    """The post-attention norm + MLP of a Qwen3.5 decoder layer
    (qwen3_5.py:200-204) on the HIP path: add + RMSNorm + gate_up + SiLU in
    one launch (the prologue kernel + row-scaled GEMM at M = 100), then
    down_proj; captured in a HIP graph, every replay equals eager execution;
    the new residual equals the reference norm's, the output stays close to
    the torch path."""
    gen = torch.Generator().manual_seed(90 + m)
    norm = _norm(gen)
    mlp = Lyr.Qwen35MLP(1024, 3584)
    _init(mlp.gate_up_proj, gen)
    _init(mlp.down_proj, gen)
    mlp = mlp.to(DEV, torch.bfloat16)
    mlp.gemm_backend = "hip"
    h_static = torch.zeros(m, 1024, dtype=torch.bfloat16, device=DEV)
    r_static = torch.zeros(m, 1024, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mlp.forward_add_norm(h_static, r_static, norm)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_static, res_static = mlp.forward_add_norm(h_static, r_static, norm)
    for step in range(3):
        h = torch.randn(m, 1024, generator=gen).bfloat16().to(DEV)
        r = torch.randn(m, 1024, generator=gen).bfloat16().to(DEV)
        h_static.copy_(h)
        r_static.copy_(r)
        graph.replay()
        torch.cuda.synchronize()
        eager, eager_res = mlp.forward_add_norm(h, r, norm)
        torch.cuda.synchronize()
        assert torch.equal(y_static, eager) and torch.equal(res_static, eager_res), f"replay {step}"
    mlp.gemm_backend = "torch"
    ref, ref_res = mlp.forward_add_norm(h, r, norm)
    assert torch.equal(eager_res, ref_res)
    assert orc.rel_frobenius(eager.double().cpu().numpy(), ref.double().cpu().numpy()) <= 1e-2


@pytest.mark.parametrize("m", [1, 32, 300])
@torch.inference_mode()
def test_gdn_forward_add_norm_hip(m):
    """The input norm of a linear-attention layer and the merged GDN
    projection (qwen3_5.py:157-163) with the norm inside the GEMM."""
    gen = torch.Generator().manual_seed(95 + m)
    norm = _norm(gen)
    proj = _init(Lyr.GdnInputProjection(1024, 16, 16, 128, 128), gen).to(DEV, torch.bfloat16)
    h = torch.randn(m, 1024, generator=gen).bfloat16().to(DEV)
    r = torch.randn(m, 1024, generator=gen).bfloat16().to(DEV)
    proj.gemm_backend = "hip"
    parts, res = proj.forward_add_norm(h, r, norm)
    proj.gemm_backend = "torch"
    ref_parts, ref_res = proj.forward_add_norm(h, r, norm)
    torch.cuda.synchronize()
    assert torch.equal(res, ref_res)
    got = torch.cat(parts, -1).double().cpu().numpy()
    ref = torch.cat(ref_parts, -1).double().cpu().numpy()
    assert got.shape == (m, 8224) and orc.rel_frobenius(got, ref) <= 1e-2


@pytest.mark.parametrize("m", [1, 8, 32, 300])
@torch.inference_mode()
def test_o_proj_forward_gated_hip(m):
    """Qwen3.5 o_proj with the output gate (qwen3_5.py:81-96: 8 heads of 256,
    gate = the second half of each head of q_proj's output): the layer on
    the HIP path equals nanovllm::gemm_gated bit for bit and stays close to
    `output * torch.sigmoid(gate)` + F.linear."""
    gen = torch.Generator().manual_seed(99 + m)
    o = _init(Lyr.RowParallelLinear(2048, 1024), gen).to(DEV, torch.bfloat16)
    attn = torch.randn(m, 8, 256, generator=gen).bfloat16().to(DEV)
    q_gate = torch.randn(m, 8, 512, generator=gen).bfloat16().to(DEV)
    gate = q_gate.chunk(2, -1)[1]
    o.gemm_backend = "hip"
    y = o.forward_gated(attn, gate)
    want = PKG.kernels.gemm_gated(attn, gate, o.weight)
    o.gemm_backend = "torch"
    ref = o.forward_gated(attn, gate)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    assert orc.rel_frobenius(y.double().cpu().numpy(), ref.double().cpu().numpy()) <= 1e-2
