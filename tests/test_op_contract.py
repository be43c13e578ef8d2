"""CPU tests of the torch op boundary: registration, fake (meta) shapes, the
argument contract and the torch | hip | auto backend switch (patterns of the
reference's tests/kernels/test_custom_add.py:36-46 and
tests/kernels/test_gdn_decode_dispatch.py:48-64)."""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import importlib

from conftest import PKG  # noqa: F401  (registers the package)

G = importlib.import_module("inference_systems_amd.kernels.gemm")


def test_ops_registered():
    assert hasattr(torch.ops.nanovllm, "gemm")
    assert hasattr(torch.ops.nanovllm, "gemm_kn")
    schema = str(torch.ops.nanovllm.gemm.default._schema)
    assert "Tensor a" in schema and "Tensor w" in schema and "ScalarType? out_dtype=None" in schema


@pytest.mark.parametrize("out_dtype", [None, torch.float32])
def test_fake_impl_shapes_on_meta(out_dtype):
    a = torch.empty((3, 5, 64), dtype=torch.bfloat16, device="meta")
    w = torch.empty((96, 64), dtype=torch.bfloat16, device="meta")
    out = torch.ops.nanovllm.gemm(a, w, out_dtype)
    assert out.shape == (3, 5, 96)
    assert out.dtype == (torch.bfloat16 if out_dtype is None else out_dtype)
    b = torch.empty((64, 40), dtype=torch.float32, device="meta")
    out = torch.ops.nanovllm.gemm_kn(torch.empty((7, 64), device="meta"), b)
    assert out.shape == (7, 40) and out.dtype == torch.float32


_REGISTRATION_PROBE = r"""
import json, sys
sys.path.insert(0, {root!r})
import torch
import __graft_entry__ as g
g.load_package()
import importlib
G = importlib.import_module("inference_systems_amd.kernels.gemm")
msgs = []
for op in (torch.ops.nanovllm.gemm, torch.ops.nanovllm.gemm_kn):
    try:
        op(torch.randn(4, 8, dtype=torch.bfloat16), torch.randn(8, 8, dtype=torch.bfloat16))
    except RuntimeError as exc:
        msgs.append(str(exc).splitlines()[0])
print(json.dumps({{"registration": G.REGISTRATION,
                  "schemas": [str(torch.ops.nanovllm.gemm.default._schema),
                              str(torch.ops.nanovllm.gemm_kn.default._schema)],
                  "cpu_messages": msgs}}))
"""


def _registration_probe(choice):
    import json
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    env = dict(os.environ)
    env.pop("NANOVLLM_GEMM_LIB", None)
    if choice is None:
        env.pop(G.OPS_ENV, None)
    else:
        env[G.OPS_ENV] = choice
    proc = subprocess.run([sys.executable, "-c", _REGISTRATION_PROBE.format(root=root)], env=env,
                          capture_output=True, text=True, timeout=300)
    return proc, (json.loads(proc.stdout.strip().splitlines()[-1]) if proc.returncode == 0 else None)


def test_registrations_share_schema_and_messages():
    """nanovllm::gemm / gemm_kn registered from C++ (TORCH_LIBRARY, the
    default when built) and from Python (custom_op over ctypes) have the
    same schemas and reject CPU operands with the same message; with the
    C++ library built, it is the default."""
    assert G.TORCH_OPS_LIB.is_file(), "libnanovllm_torch_ops.so is not built"
    _, default = _registration_probe(None)
    _, cpp = _registration_probe("torch_library")
    _, py = _registration_probe("custom_op")
    assert default["registration"] == "torch_library"
    assert cpp["registration"] == "torch_library" and py["registration"] == "custom_op"
    assert cpp["schemas"] == py["schemas"]
    assert cpp["cpu_messages"] == py["cpu_messages"] == ["nanovllm::gemm: a and w must be CUDA (HIP) tensors"] * 2


def test_registration_choice_is_validated():
    proc, _ = _registration_probe("cuda_graphs")
    assert proc.returncode != 0 and "NANOVLLM_GEMM_OPS must be one of" in proc.stderr


def test_op_rejects_cpu_tensors():
    a = torch.randn(4, 8, dtype=torch.bfloat16)
    w = torch.randn(6, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="must be CUDA"):
        torch.ops.nanovllm.gemm(a, w)


def test_contract_reason_cpu():
    a = torch.randn(4, 8)
    assert G.contract_reason(a, torch.randn(6, 8)) == "a and w must be CUDA (HIP) tensors"


def test_backend_validation(monkeypatch):
    assert G.validate_gemm_backend(" HIP ") == "hip"
    with pytest.raises(ValueError, match="GEMM backend must be one of"):
        G.validate_gemm_backend("cublas")
    monkeypatch.setenv(G.BACKEND_ENV, "auto")
    assert G.default_backend() == "auto"
    monkeypatch.delenv(G.BACKEND_ENV)
    assert G.default_backend() == "torch"


def test_linear_backends_on_cpu_tensors():
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(3, 16, generator=gen)
    w = torch.randn(8, 16, generator=gen)
    b = torch.randn(8, generator=gen)
    ref = F.linear(x, w, b)
    assert torch.equal(G.linear(x, w, b, backend="torch"), ref)
    # auto: CPU tensors are outside the HIP op's contract -> F.linear
    assert torch.equal(G.linear(x, w, b, backend="auto"), ref)
    with pytest.raises(RuntimeError, match="HIP GEMM backend is unavailable: a and w must be CUDA"):
        G.linear(x, w, b, backend="hip")
    out = G.linear(x.bfloat16(), w.bfloat16(), None, out_dtype=torch.float32, backend="torch")
    assert out.dtype == torch.float32


def test_sample_op_registered_and_fake_shapes():
    """nanovllm::gemm_sample: registered with (a, w, temperatures, seed,
    offset) and a meta implementation giving (int64 tokens, fp32 scores)
    over the leading dims of a."""
    schema = str(torch.ops.nanovllm.gemm_sample.default._schema)
    assert "Tensor temperatures" in schema and "seed" in schema and "offset" in schema
    a = torch.empty((2, 3, 64), dtype=torch.bfloat16, device="meta")
    w = torch.empty((500, 64), dtype=torch.bfloat16, device="meta")
    t = torch.empty((2, 3), dtype=torch.float32, device="meta")
    tokens, scores = torch.ops.nanovllm.gemm_sample(a, w, t, 1, 2)
    assert tokens.shape == (2, 3) and tokens.dtype == torch.int64
    assert scores.shape == (2, 3) and scores.dtype == torch.float32


def test_sample_contract_reasons_and_backends():
    """The sampled head's contract on CPU tensors, and sample_linear's torch
    backend (the reference Sampler on F.linear's logits)."""
    a = torch.randn(4, 16, dtype=torch.bfloat16)
    w = torch.randn(10, 16, dtype=torch.bfloat16)
    t = torch.zeros(4)
    assert G.sample_contract_reason(a, w, t) == "a and w must be CUDA (HIP) tensors"
    tokens, scores = G.sample_linear(a, w, t, 1, 2, backend="auto")
    assert scores is None and torch.equal(tokens, F.linear(a, w).float().argmax(-1))
    with pytest.raises(RuntimeError, match="HIP GEMM backend is unavailable"):
        G.sample_linear(a, w, t, 1, 2, backend="hip")
