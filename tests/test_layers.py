"""CPU tests of the nano-vLLM layer mirrors (inference-systems_amd/layers).

Weight loading and tensor-parallel sharding must match the reference layers
(nanovllm/layers/linear.py:12-156, embed_head.py:45-66); on CPU tensors the
``auto`` backend routes to F.linear, so outputs compare exactly with an
unsharded F.linear.  The 2-rank case follows the reference's gloo pattern
(tests/test_qwen35_tp.py:26-31, 125-158)."""
from __future__ import annotations

import importlib
import os
import tempfile

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp
import torch.nn.functional as F

from conftest import PKG

Lyr = PKG.layers


def _full_weights(seed=0, k=64, n=96):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, k, generator=g), torch.randn(n, generator=g)


def test_single_process_layers_match_f_linear():
    w, b = _full_weights()
    x = torch.randn(5, 64)
    for cls in (Lyr.ReplicatedLinear, Lyr.ColumnParallelLinear):
        layer = cls(64, 96, bias=True)
        layer.weight.weight_loader(layer.weight, w)
        layer.bias.weight_loader(layer.bias, b)
        layer.gemm_backend = "auto"
        assert torch.equal(layer(x), F.linear(x, w, b))
    row = Lyr.RowParallelLinear(96, 64, bias=True)
    wr, br = torch.randn(64, 96), torch.randn(64)
    row.weight.weight_loader(row.weight, wr)
    row.bias.weight_loader(row.bias, br)
    row.gemm_backend = "torch"
    y = torch.randn(3, 96)
    assert torch.equal(row(y), F.linear(y, wr, br))


def test_merged_and_qkv_loaders():
    merged = Lyr.MergedColumnParallelLinear(32, [48, 48])
    g0, g1 = torch.randn(48, 32), torch.randn(48, 32)
    merged.weight.weight_loader(merged.weight, g0, 0)
    merged.weight.weight_loader(merged.weight, g1, 1)
    assert torch.equal(merged.weight.data, torch.cat([g0, g1]))
    qkv = Lyr.QKVParallelLinear(32, head_size=8, total_num_heads=4, total_num_kv_heads=2)
    q, k, v = torch.randn(32, 32), torch.randn(16, 32), torch.randn(16, 32)
    for shard, t in (("q", q), ("k", k), ("v", v)):
        qkv.weight.weight_loader(qkv.weight, t, shard)
    assert torch.equal(qkv.weight.data, torch.cat([q, k, v]))
    qkv.gemm_backend = "auto"
    x = torch.randn(2, 32)
    assert torch.equal(qkv(x), F.linear(x, torch.cat([q, k, v])))


def test_lm_head_last_indices_and_logits_dtype():
    """The head's logits are the reference's (F.linear in the model dtype,
    embed_head.py:61) unless fp32 logits are asked for."""
    head = Lyr.ParallelLMHead(100, 16)
    w = torch.randn(100, 16).bfloat16()
    head.weight.data = torch.empty(100, 16, dtype=torch.bfloat16)
    head.weight.weight_loader(head.weight, w)
    head.gemm_backend = "auto"
    x = torch.randn(7, 16).bfloat16()
    last = torch.tensor([2, 6])
    logits = head(x, last)
    assert logits.shape == (2, 100) and logits.dtype == torch.bfloat16
    assert torch.equal(logits, F.linear(x[last], w))
    head.logits_dtype = torch.float32
    logits = head(x, last)
    assert logits.dtype == torch.float32
    assert torch.equal(logits, F.linear(x[last], w).float())


def test_gemm_linear_module():
    m = Lyr.GemmLinear(16, 8)
    m.gemm_backend = "auto"
    x = torch.randn(3, 16)
    assert torch.equal(m(x), F.linear(x, m.weight, m.bias))


def _gdn_weights(hidden=8, key_heads=2, value_heads=4, kdim=3, vdim=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    conv = 2 * key_heads * kdim + value_heads * vdim
    return {"qkv": torch.randn(conv, hidden, generator=g), "z": torch.randn(value_heads * vdim, hidden, generator=g),
            "b": torch.randn(value_heads, hidden, generator=g), "a": torch.randn(value_heads, hidden, generator=g)}


@pytest.mark.parametrize("dims", [(8, 2, 4, 3, 2), (64, 4, 8, 16, 8)])
def test_gdn_projection_matches_four_linears(dims):
    """One GEMM over the merged weight gives the four projections of
    gated_delta_net.py:192-195, in the order qkv, z, b, a."""
    hidden, kh, vh, kd, vd = dims
    full = _gdn_weights(hidden, kh, vh, kd, vd)
    proj = Lyr.GdnInputProjection(hidden, kh, vh, kd, vd)
    for sid, w in full.items():
        proj.weight.weight_loader(proj.weight, w, sid)
    assert proj.weight.shape == (2 * kh * kd + 2 * vh * vd + 2 * vh, hidden)
    proj.gemm_backend = "auto"
    x = torch.randn(5, hidden)
    outs = proj(x)
    assert [o.shape[-1] for o in outs] == [2 * kh * kd + vh * vd, vh * vd, vh, vh]
    for out, sid in zip(outs, ("qkv", "z", "b", "a")):
        torch.testing.assert_close(out, F.linear(x, full[sid]))
    # several rows: views by default; contiguous outputs on request, as
    # gdn_decode_core's CUDA path asks (nanovllm/kernels/gdn.py:186)
    assert not outs[0].is_contiguous()
    parts = proj(x, contiguous=True)
    assert all(p.is_contiguous() for p in parts)
    for part, sid in zip(parts, ("qkv", "z", "b", "a")):
        torch.testing.assert_close(part, F.linear(x, full[sid]))
    assert all(o.is_contiguous() for o in proj(x[:1]))
    with pytest.raises(ValueError, match="shard id"):
        proj.weight.weight_loader(proj.weight, full["z"], "v")


def test_lm_head_greedy_matches_argmax_of_logits():
    """Sampler's greedy branch: argmax of the fp32 logits, first index on ties
    (two vocabulary rows are duplicated so their logits tie exactly)."""
    head = Lyr.ParallelLMHead(50, 16)
    w = torch.randn(50, 16, generator=torch.Generator().manual_seed(4))
    w[31] = w[7]
    head.weight.weight_loader(head.weight, w)
    head.gemm_backend = "auto"
    x = torch.randn(6, 16)
    x[2] = w[7] * 3.0           # row 2 prefers token 7, tied with token 31
    tokens, values = head.greedy(x)
    logits = head(x)
    assert torch.equal(tokens, logits.argmax(-1))
    assert int(tokens[2]) == 7
    torch.testing.assert_close(values, logits.gather(-1, tokens[:, None]).squeeze(-1))
    t2, _ = head.greedy(torch.randn(9, 16), last_indices=torch.tensor([0, 8]))
    assert t2.shape == (2,)


def test_lm_head_sample_torch_path():
    """ParallelLMHead.sample off the HIP path runs the reference Sampler on
    the fp32 logits: greedy rows (temperature <= 1e-10) are the greedy
    tokens, sampled rows valid token ids, and no scores."""
    head = Lyr.ParallelLMHead(50, 16)
    head.weight.weight_loader(head.weight, torch.randn(50, 16, generator=torch.Generator().manual_seed(6)))
    head.gemm_backend = "auto"
    x = torch.randn(8, 16, generator=torch.Generator().manual_seed(7))
    temps = torch.tensor([0.0, 1.0, 1e-10, 0.7, 0.0, 2.0, 0.0, 0.3])
    tokens, scores = head.sample(x, temps, seed=1, offset=2)
    greedy_tokens, _ = head.greedy(x)
    greedy = temps <= 1e-10
    assert scores is None and tokens.dtype == torch.int64 and tokens.shape == (8,)
    assert torch.equal(tokens[greedy], greedy_tokens[greedy])
    assert ((tokens >= 0) & (tokens < 50)).all()
    torch.manual_seed(0)
    many = torch.stack([head.sample(x[1:2], temps[1:2], 1, 2)[0] for _ in range(2000)]).flatten()
    p = torch.softmax(head(x[1:2]).float(), -1).flatten()
    top = int(p.argmax())
    assert abs(float((many == top).float().mean()) - float(p[top])) < 0.05


def test_qwen35_mlp_matches_reference_composition():
    """down_proj(SiluAndMul(gate_up_proj(x))) of models/qwen3_5.py:117-118; on
    CPU tensors the auto backend takes the reference composition."""
    mlp = Lyr.Qwen35MLP(32, 48)
    g = torch.Generator().manual_seed(3)
    wg, wu, wd = torch.randn(48, 32, generator=g), torch.randn(48, 32, generator=g), torch.randn(32, 48, generator=g)
    mlp.gate_up_proj.weight.weight_loader(mlp.gate_up_proj.weight, wg, 0)
    mlp.gate_up_proj.weight.weight_loader(mlp.gate_up_proj.weight, wu, 1)
    mlp.down_proj.weight.weight_loader(mlp.down_proj.weight, wd)
    x = torch.randn(5, 32, generator=g)
    ref = F.linear(F.silu(F.linear(x, wg)) * F.linear(x, wu), wd)
    for backend in ("torch", "auto"):
        mlp.gemm_backend = backend
        assert mlp.gate_up_proj.gemm_backend == backend and mlp.down_proj.gemm_backend == backend
        torch.testing.assert_close(mlp(x), ref)
    with pytest.raises(ValueError, match="SiLU"):
        Lyr.Qwen35MLP(32, 48, hidden_act="gelu")
    mlp.gemm_backend = "hip"
    with pytest.raises(RuntimeError, match="CUDA"):
        mlp(x)


def test_qwen35_rmsnorm_mirror():
    """Qwen3_5RMSNorm (layernorm.py:110-142): zero-centred scale, 1 + w in
    fp32; with a residual, (round(norm(x + r)), round(x + r))."""
    g = torch.Generator().manual_seed(4)
    norm = Lyr.Qwen35RMSNorm(16, eps=1e-6)
    x = torch.randn(3, 16, generator=g).bfloat16()
    r = torch.randn(3, 16, generator=g).bfloat16()
    # w = 0: plain RMSNorm
    x32 = x.float()
    want = (x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + 1e-6)).bfloat16()
    assert torch.equal(norm(x), want)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(16, generator=g) * 0.1)
    y, new_r = norm(x, r)
    s = x.float() + r.float()
    assert torch.equal(new_r, s.bfloat16())
    want = (s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + norm.weight.float())).bfloat16()
    assert torch.equal(y, want)


def test_forward_add_norm_and_gated_torch_paths():
    """The fused entry points of the layers on the torch backend are the
    reference compositions: norm then MLP / merged projection
    (qwen3_5.py:157-163, 200-204), o_proj of x * sigmoid(gate) (:95-96)."""
    g = torch.Generator().manual_seed(6)
    norm = Lyr.Qwen35RMSNorm(32)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(32, generator=g) * 0.1)
    mlp = Lyr.Qwen35MLP(32, 48)
    for p_ in mlp.parameters():
        with torch.no_grad():
            p_.copy_(torch.randn(p_.shape, generator=g) * 0.1)
    h, r = torch.randn(5, 32, generator=g), torch.randn(5, 32, generator=g)
    for backend in ("torch", "auto"):
        mlp.gemm_backend = backend
        out, new_r = mlp.forward_add_norm(h, r, norm)
        normed, want_r = norm(h, r)
        torch.testing.assert_close(out, mlp(normed))
        assert torch.equal(new_r, want_r)
    proj = Lyr.GdnInputProjection(32, 2, 2, 4, 4)
    with torch.no_grad():
        proj.weight.copy_(torch.randn(proj.weight.shape, generator=g) * 0.1)
    proj.gemm_backend = "auto"
    parts, new_r = proj.forward_add_norm(h, r, norm)
    for got, want in zip(parts, proj(norm(h, r)[0])):
        torch.testing.assert_close(got, want)
    o = Lyr.RowParallelLinear(16, 24)
    with torch.no_grad():
        o.weight.copy_(torch.randn(24, 16, generator=g))
    o.gemm_backend = "auto"
    attn = torch.randn(5, 2, 8, generator=g)
    q_gate = torch.randn(5, 2, 16, generator=g)
    gate = q_gate.chunk(2, -1)[1]
    torch.testing.assert_close(o.forward_gated(attn, gate),
                               F.linear((attn * torch.sigmoid(gate)).flatten(1), o.weight))


def _tp_worker(rank, world, init_file, result_file):
    dist.init_process_group("gloo", init_method=f"file://{init_file}", rank=rank, world_size=world)
    try:
        torch.manual_seed(0)
        k, n, m = 32, 64, 6
        w1, b1 = torch.randn(n, k), torch.randn(n)
        w2, b2 = torch.randn(k, n), torch.randn(k)
        x = torch.randn(m, k)
        col = Lyr.ColumnParallelLinear(k, n, bias=True)
        col.weight.weight_loader(col.weight, w1)
        col.bias.weight_loader(col.bias, b1)
        row = Lyr.RowParallelLinear(n, k, bias=True)
        row.weight.weight_loader(row.weight, w2)
        row.bias.weight_loader(row.bias, b2)
        for mod in (col, row):
            mod.gemm_backend = "auto"
        y = row(col(x))
        ref = F.linear(F.linear(x, w1, b1), w2, b2)
        # sharded partial sums + all_reduce reorder the fp32 sum: tolerance 1e-4
        ok = torch.allclose(y, ref, rtol=1e-4, atol=1e-4)
        head = Lyr.ParallelLMHead(40, k)
        wh = torch.randn(40, k)
        head.weight.weight_loader(head.weight, wh)
        head.gemm_backend = "auto"
        logits = head(x)
        if rank == 0:
            ok = ok and torch.allclose(logits, F.linear(x, wh), rtol=1e-6, atol=1e-6)
        else:
            ok = ok and logits is None
        # Merged GDN projection: the per-rank rows the reference's loaders
        # pick (tests/test_qwen35_tp.py:39-55 with 2 key heads of 3 and 4
        # value heads of 2: q, k, v each cut from its own third).
        proj = Lyr.GdnInputProjection(8, 2, 4, 3, 2)
        full_qkv = torch.arange(20 * 8, dtype=torch.float32).reshape(20, 8)
        full_z = torch.arange(8 * 8, dtype=torch.float32).reshape(8, 8)
        full_b = torch.arange(4 * 8, dtype=torch.float32).reshape(4, 8) * 2
        full_a = torch.arange(4 * 8, dtype=torch.float32).reshape(4, 8) * 3
        for sid, wt in (("qkv", full_qkv), ("z", full_z), ("b", full_b), ("a", full_a)):
            proj.weight.weight_loader(proj.weight, wt, sid)
        want = torch.cat((full_qkv[rank * 3:(rank + 1) * 3], full_qkv[6 + rank * 3:6 + (rank + 1) * 3],
                          full_qkv[12 + rank * 4:12 + (rank + 1) * 4], full_z[rank * 4:(rank + 1) * 4],
                          full_b[rank * 2:(rank + 1) * 2], full_a[rank * 2:(rank + 1) * 2]), dim=0)
        ok = ok and proj.conv_dim == 10 and torch.equal(proj.weight.data, want)
        proj.gemm_backend = "auto"
        xg = torch.randn(3, 8)
        ok = ok and torch.allclose(torch.cat(proj(xg), dim=-1), F.linear(xg, want), rtol=1e-6, atol=1e-5)
        # Greedy head across vocabulary shards: the best token overall, the
        # lower shard on a tie (token 5 of rank 0 and token 25 of rank 1
        # have equal logits).
        gh = Lyr.ParallelLMHead(40, k)
        wt = torch.randn(40, k, generator=torch.Generator().manual_seed(12))
        wt[25] = wt[5]
        gh.weight.weight_loader(gh.weight, wt)
        gh.gemm_backend = "auto"
        xt = torch.randn(4, k, generator=torch.Generator().manual_seed(13))
        xt[1] = wt[5] * 2.0
        gt, gv = gh.greedy(xt)
        if rank == 0:
            full = F.linear(xt, wt)
            ok = ok and torch.equal(gt, full.argmax(-1)) and int(gt[1]) == 5
            ok = ok and torch.allclose(gv, full.max(-1).values, rtol=1e-6, atol=1e-6)
        else:
            ok = ok and gt is None and gv is None
        # Sampled head across shards off the HIP path: the logits are
        # gathered to rank 0, which runs the reference Sampler; greedy rows
        # (temperature 0) give the greedy tokens.
        st, ss = gh.sample(xt, torch.zeros(4), seed=3, offset=4)
        if rank == 0:
            ok = ok and ss is None and torch.equal(st, F.linear(xt, wt).argmax(-1))
        else:
            ok = ok and st is None and ss is None
        # o_proj with the output gate: each rank holds its heads' columns of
        # W and its heads of the attention output and the gate (the head split
        # of the reference's tensor parallelism); the all-reduce adds them.
        og = torch.Generator().manual_seed(14)
        w_o = torch.randn(k, 4 * 8, generator=og)
        attn = torch.randn(m, 4, 8, generator=og)
        gate = torch.randn(m, 4, 16, generator=og).chunk(2, -1)[1]
        o = Lyr.RowParallelLinear(4 * 8, k)
        o.weight.weight_loader(o.weight, w_o)
        o.gemm_backend = "auto"
        mine = slice(rank * 2, rank * 2 + 2)
        yo = o.forward_gated(attn[:, mine].contiguous(), gate[:, mine])
        ok = ok and torch.allclose(yo, F.linear((attn * torch.sigmoid(gate)).flatten(1), w_o), rtol=1e-4, atol=1e-4)
        with open(f"{result_file}.{rank}", "w") as fh:
            fh.write("ok" if ok else "mismatch")
    finally:
        dist.destroy_process_group()


def test_tensor_parallel_two_ranks_gloo():
    with tempfile.TemporaryDirectory() as tmp:
        init_file = os.path.join(tmp, "init")
        result = os.path.join(tmp, "result")
        # spawn, not fork: earlier tests in this process may have started
        # torch's OpenMP pool, and a forked child entering it can deadlock.
        mp.start_processes(_tp_worker, args=(2, init_file, result), nprocs=2, start_method="spawn")
        for r in range(2):
            assert open(f"{result}.{r}").read() == "ok", f"rank {r}"


def test_sample_seed_and_offset_wrap_to_64_bits():
    """Seeds and offsets reach the C ABI as their low 64 bits, through the
    op schema's signed int."""
    G = importlib.import_module(PKG.__name__ + ".kernels.gemm")
    assert G._as_i64(5) == 5
    assert G._as_i64(-1) == -1
    assert G._as_i64((1 << 64) - 1) == -1
    assert G._as_i64(1 << 63) == -(1 << 63)
    assert G._as_i64((1 << 64) + 7) == 7
