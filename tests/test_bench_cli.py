"""bench.py's contract on the CPU: more than one GPU is refused with a
message, and the shape-matrix inputs are the reference's generators
(gemm_bench.cu:296-305, restated in the oracle)."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import torch

from oracle import gemm_oracle as orc

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_matrix_inputs_are_the_reference_generators():
    for m, n, k in ((1, 7, 64), (16, 33, 130), (5, 4, 3)):
        a, b = bench.reference_inputs(torch, m, n, k)
        assert np.array_equal(a.numpy() * 32, orc.kat_bench_a_int(m, k).astype(np.float32))
        assert np.array_equal(b.numpy() * 32, orc.kat_bench_b_int(k, n).astype(np.float32))
        # exact in both half formats
        for dt in (torch.float16, torch.bfloat16):
            assert torch.equal(a.to(dt).float(), a) and torch.equal(b.to(dt).float(), b)


def test_vendor_tuned_cases_are_workloads():
    """Every row of `bench.py --vendor-tuned` is a workload of the table at one
    of its M values, with a single-call torch equivalent of the same output
    dtype (the fp32-logit LM head has none)."""
    W = bench.__dict__.get("VENDOR_TUNED_CASES")
    import __graft_entry__
    wl = __graft_entry__.load_package().workloads.WORKLOADS
    assert W
    for name, m in W:
        assert name in wl and m in wl[name].ms
        assert wl[name].dtype_out == wl[name].dtype_in


def test_stability_cases_read_every_timed_row():
    """`bench.py --stability` reads the headline, its W-from-HBM row, every
    decode row, every other workload and the eager call of a bench line,
    with torch's time where the line has one."""
    line = {
        "config": {"workload": "bf16_prefill_2048x4096x1024"}, "ms_per_step": 0.0175,
        "vendor_torch_linear": {"us": 20.5}, "headline_w_from_hbm": {"us": 21.0},
        "decode_bf16_n6144_k1024": [{"m": 1, "us": 3.8, "torch_gpu_us": 6.0}, {"m": 32, "us": 5.6}],
        "other_workloads": [{"workload": "fp32_square_1024", "m": 1024, "us": 19.4, "torch_gpu_us": 18.5}],
        "eager_call_overhead": {"rows": {"nanovllm::gemm": {"host_us": 5.3}, "F.linear": {"host_us": 19.5}}},
    }
    cases = list(bench._stability_cases(line))
    assert cases == [
        ("headline bf16_prefill_2048x4096x1024", 17.5, 20.5),
        ("headline, W rotated from HBM", 21.0, None),
        ("bf16_decode_n6144_k1024 M=1", 3.8, 6.0),
        ("bf16_decode_n6144_k1024 M=32", 5.6, None),
        ("fp32_square_1024 M=1024", 19.4, 18.5),
        ("eager call host time, nanovllm::gemm M=1", 5.3, 19.5),
    ]


def test_decode_sweep_shapes_parse():
    """`--decode-sweep-shapes` takes N x K pairs; K must be a positive
    multiple of 8 (the decode kernels' 16-byte chunks)."""
    assert bench.parse_shapes("151936x1024") == ((151936, 1024),)
    assert bench.parse_shapes("6144x1024,1024X3584") == ((6144, 1024), (1024, 3584))
    import pytest
    for bad in ("6144x1000x2", "6144x1020", "0x1024", "6144"):
        with pytest.raises(ValueError):
            bench.parse_shapes(bad)
