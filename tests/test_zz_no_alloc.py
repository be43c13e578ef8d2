"""GPU tests of nanovllm_gemm_argmax_noalloc, the greedy LM head without a
workspace (its per-workgroup keys live in the library's device scratch
array), called through the C ABI and checked bit for bit against
nanovllm_gemm_argmax with a caller workspace on the same inputs."""
from __future__ import annotations

import pytest
import torch

from conftest import PKG

pytestmark = pytest.mark.gpu

L = PKG._lib
DEV = torch.device("cuda:0")
CODE = {torch.float16: L.F16, torch.bfloat16: L.BF16}


def _say(msg):
    print(msg, flush=True)


def _inputs(m, n, k, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    a = torch.randn((m, k), generator=gen).to(dtype).to(DEV)
    w = (torch.randn((n, k), generator=gen) * 0.05).to(dtype).to(DEV)
    return a, w


def _noalloc(a, w, logit):
    m, k = a.shape
    n = w.shape[0]
    tokens = torch.full((m,), -1, dtype=torch.int64, device=DEV)
    values = torch.full((m,), float("nan"), dtype=torch.float32, device=DEV)
    rc = L.load().nanovllm_gemm_argmax_noalloc(a.data_ptr(), w.data_ptr(), tokens.data_ptr(), values.data_ptr(),
                                               m, n, k, k, k, CODE[a.dtype], logit,
                                               torch.cuda.current_stream().cuda_stream)
    L.check(rc, "nanovllm_gemm_argmax_noalloc")
    return tokens, values


def _with_workspace(a, w, logit):
    m, k = a.shape
    n = w.shape[0]
    tokens = torch.empty((m,), dtype=torch.int64, device=DEV)
    values = torch.empty((m,), dtype=torch.float32, device=DEV)
    need = L.argmax_workspace_bytes(m, n, k, k, k, CODE[a.dtype])
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    L.argmax_raw(a.data_ptr(), w.data_ptr(), tokens.data_ptr(), values.data_ptr(), m, n, k, k, k, CODE[a.dtype],
                 logit, ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    return tokens, values


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("rank", ["model", "f32"])
def test_noalloc_equals_workspace_entry(dtype, rank):
    """Two calls in a row on one device, the second smaller: the Qwen3.5 LM
    head at M = 300 (mfma_staged, 300 x 1187 keys) then M = 5 on a ragged
    vocabulary (splitk_decode); each equals the workspace entry point's
    tokens and values exactly (the second call reads no stale key of the
    first)."""
    logit = CODE[dtype] if rank == "model" else L.F32
    for m, n, k, seed in ((300, 151936, 1024, 1), (5, 70001, 256, 2)):
        _say(f"noalloc {rank} {dtype} M={m} N={n} K={k}")
        a, w = _inputs(m, n, k, dtype, seed)
        t0, v0 = _noalloc(a, w, logit)
        t1, v1 = _with_workspace(a, w, logit)
        torch.cuda.synchronize()
        assert torch.equal(t0, t1) and torch.equal(v0, v1), (m, n, k)
        assert bool((t0 >= 0).all()) and bool((t0 < n).all())


def test_noalloc_graph_replay():
    """Captured in a HIP graph (no allocation inside the capture) and
    replayed with new inputs and eager work between replays: every replay
    equals the eager call."""
    m, n, k = 32, 151936, 1024
    a, w = _inputs(m, n, k, torch.bfloat16, 3)
    a_static = a.clone()
    tokens = torch.empty((m,), dtype=torch.int64, device=DEV)
    values = torch.empty((m,), dtype=torch.float32, device=DEV)
    lib = L.load()

    def call():
        rc = lib.nanovllm_gemm_argmax_noalloc(a_static.data_ptr(), w.data_ptr(), tokens.data_ptr(),
                                              values.data_ptr(), m, n, k, k, k, L.BF16, L.BF16,
                                              torch.cuda.current_stream().cuda_stream)
        L.check(rc, "nanovllm_gemm_argmax_noalloc")

    _say("noalloc graph replay")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()                        # first call on the device, outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    gen = torch.Generator().manual_seed(9)
    for step in range(3):
        a_static.copy_(torch.randn((m, k), generator=gen).bfloat16().to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        t_r, v_r = tokens.clone(), values.clone()
        t_e, v_e = _with_workspace(a_static, w, L.BF16)
        torch.cuda.synchronize()
        assert torch.equal(t_r, t_e) and torch.equal(v_r, v_e), f"replay {step}"


def test_noalloc_rejects_problems_beyond_its_scratch():
    """A problem whose keys exceed the 8 MiB scratch is refused with a clear
    message before anything is launched; the output is left untouched."""
    m, n, k = 1024, 151936, 1024
    a, w = _inputs(8, 64, k, torch.bfloat16, 4)
    tokens = torch.full((m,), -7, dtype=torch.int64, device=DEV)
    rc = L.load().nanovllm_gemm_argmax_noalloc(a.data_ptr(), w.data_ptr(), tokens.data_ptr(), None, m, n, k, k, k,
                                               L.BF16, L.BF16, torch.cuda.current_stream().cuda_stream)
    assert rc == L.EINVAL and "scratch" in L.last_error()
    torch.cuda.synchronize()
    assert bool((tokens == -7).all())
