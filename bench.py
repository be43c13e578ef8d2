#!/usr/bin/env python3
"""Benchmark of the shape-aware GEMM path on one MI355X.

Headline: the BF16 prefill projection C[2048,4096] = A[2048,1024] W[4096,1024]^T
(bf16 out, fp32 accumulate) on the kernel the selection table picks.  A step
is one GEMM over resident inputs.  The K timed steps are launched back to
back on one stream and timed with HIP events on that stream, the pattern of
the reference's benchmark_ms (cuda_kernels/gemm/src/gemm_bench.cu:198-223);
the same K steps replayed as one HIP graph are reported beside them.  For the
short bandwidth-bound workloads (``--workload`` with a decode shape, and the
decode rows below) the graph replay is the measure, so host launch gaps are
excluded, and plain stream launches are reported beside it.

Alongside (extra keys of the same JSON line): the decode GEMMs M in
{1,4,8,16,32} x N=6144 x K=1024 with W rotated over more than twice the
256 MB Infinity Cache, the FP32 1024^3 GEMM, the FP16 down projection, the
BF16 LM head, the merged gated-delta-net input projection (one N = 8224 GEMM
against four launches), the fused epilogues and prologues against the
reference's compositions (gate_up + SiLU-and-mul, the greedy and the sampled
LM head, the gated-attention output gate before o_proj, the residual add +
RMSNorm before a projection), the bf16 rows of the reference's shape matrix
(below), torch's own GPU GEMM (hipBLASLt / rocBLAS) on the same inputs
for comparison only, and the CPU baseline (host F.linear, multi-threaded).

Prints ONE JSON line on stdout; a readable table goes to stderr.  With
``--matrix`` it instead runs the reference's own shape matrix (its Qwen3.5
shapes in fp16 and bf16, deterministic inputs, fp32 output) and prints it
as CSV, one row per shape in the columns of the reference's results file.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PEAK_MFMA_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}   # MI355X dense
PEAK_HBM_GBS = 8000.0
INFINITY_CACHE_BYTES = 256 * 2 ** 20
DEVICE_WARMUP_S = 0.3
TRAFFIC_FILE = ROOT / "profiles" / "traffic_bf16_prefill_2048x4096x1024.md"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--no-extras", action="store_true", help="headline only")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-vendor", action="store_true", help="skip the torch GPU GEMM comparison")
    p.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline sampling")
    p.add_argument("--workload", default=None,
                   help="measure this workload instead of the prefill headline (for profiling one kernel)")
    p.add_argument("--m", type=int, default=None, help="M of --workload (default: its largest)")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                   help="only run 10 device copies of MIB MiB (reference kernel for HBM counter scaling)")
    p.add_argument("--probes", action="store_true",
                   help="only run the microbenchmarks of the hardware ceilings (launch floor, streaming read, LDS "
                        "reads, global -> LDS copies, MFMA rate, clocks) and print them as one JSON line")
    p.add_argument("--decode-sweep", action="store_true",
                   help="only run every configuration of the decode kernels (rows of A and of W per workgroup, "
                        "waves, lines per wave) on the decode shapes and print them as one JSON line")
    p.add_argument("--decode-sweep-shapes", default=None, metavar="NxK[,NxK...]",
                   help="the W shapes of --decode-sweep (default: the Qwen3.5-0.8B decode shapes and 16384x1024)")
    p.add_argument("--matrix", action="store_true",
                   help="only run the reference's shape matrix (fp16 and bf16 over its Qwen3.5 shapes) and print "
                        "it as CSV")
    p.add_argument("--vendor-tuned", action="store_true",
                   help="only time torch's GPU GEMM with every hipBLASLt / rocBLAS solution searched (TunableOp) "
                        "beside its default choice and the selected kernel here, on the workloads that fit one "
                        "torch call, and print them as one JSON line")
    p.add_argument("--eager-overhead", action="store_true",
                   help="only time the host cost of one eager call (nanovllm::gemm under the registration "
                        "NANOVLLM_GEMM_OPS picks, the Linear path, the bare C ABI, F.linear) and print it as one "
                        "JSON line")
    p.add_argument("--stability", type=int, default=0, metavar="RUNS",
                   help="only run the default bench (without the CPU baseline) RUNS times, each in a fresh child "
                        "process (this process never touches the GPU), and print mean / std / min / max per "
                        "workload and the ratio to torch's GPU GEMM as one JSON line")
    p.add_argument("--data-patterns", action="store_true",
                   help="only time the prefill headline, the fp16 down projection and the LM head at M = 512, "
                        "ours and torch's GPU GEMM, on random, mantissa-free, constant and zero inputs (the "
                        "MFMA-bound kernels run at the power limit, so their speed depends on the data) and print "
                        "one JSON line")
    p.add_argument("--counter-pair", type=int, default=0, metavar="CALLS",
                   help="only call nanovllm::gemm and torch's equivalent GEMM on --workload / --m: one call of "
                        "each compared, then two rounds of CALLS calls of ours followed by CALLS of torch's (a "
                        "fixed dispatch sequence for rocprofv3 counter passes; no timing)")
    return p.parse_args()


def calibrate_copy(mib: int) -> int:
    """A plain device-to-device copy of known size: its FETCH_SIZE / WRITE_SIZE
    counters give the scale between the counters and bytes moved."""
    import torch

    n = mib * 2 ** 20 // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_each_way": n * 4, "copies": 10}), flush=True)
    return 0


class GraphTimer:
    """Captures a list of launches into one HIP graph and times a replay."""

    def __init__(self, torch, launches):
        self.torch = torch
        self.graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            launches[0]()   # first launch outside capture
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(self.graph):
            for f in launches:
                f()
        torch.cuda.synchronize()

    def time_ms(self) -> float:
        t = self.torch
        start, end = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        t.cuda.synchronize()
        start.record()
        self.graph.replay()
        end.record()
        t.cuda.synchronize()
        return start.elapsed_time(end)


def median_plain_ms(torch, launches, trials=5) -> float:
    """Median over trials of (time / launches) for the same launches issued
    one by one on the stream, without a graph (host launch cost included)."""
    for f in launches[:4]:
        f()
    torch.cuda.synchronize()
    samples = []
    for _ in range(trials):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for f in launches:
            f()
        end.record()
        torch.cuda.synchronize()
        samples.append(start.elapsed_time(end) / len(launches))
    return sorted(samples)[len(samples) // 2]


RAMP_MS = 30.0   # GPU time replayed before the trials of an extra row


def median_graph_ms(torch, launches, trials=5) -> float:
    """Median over trials of (graph replay time / launches), in ms.  The
    graph is replayed for RAMP_MS first: capture leaves the GPU idle, and
    the clocks of an idle MI355X drop."""
    timer = GraphTimer(torch, launches)
    ramp = 0.0
    while ramp < RAMP_MS:
        ramp += timer.time_ms()
    samples = sorted(timer.time_ms() / len(launches) for _ in range(trials))
    return samples[len(samples) // 2]


def read_traffic():
    """HBM bytes per launch of the headline kernel from the committed
    rocprofv3 PMC summary, or None."""
    if not TRAFFIC_FILE.is_file():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def benchmark_ms(torch, launch, warmup: int, repeats: int, trials: int = 7) -> tuple:
    """The reference's benchmark_ms (cuda_kernels/gemm/src/gemm_bench.cu:198-223):
    `warmup` launches, then the median over `trials` of (event time of
    `repeats` back-to-back launches) / repeats.  Returns (graph, plain):
    the same `repeats` launches replayed as one HIP graph (after a clock
    ramp; host launch cost excluded), and issued one by one from Python."""
    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    samples = []
    for _ in range(trials):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(repeats):
            launch()
        end.record()
        end.synchronize()
        samples.append(start.elapsed_time(end) / repeats)
    samples.sort()
    plain = samples[len(samples) // 2]
    timer = GraphTimer(torch, [launch] * repeats)
    ramp = 0.0
    while ramp < RAMP_MS:
        ramp += timer.time_ms()
    graph = sorted(timer.time_ms() / repeats for _ in range(trials))[trials // 2]
    return graph, plain


def run_probes(torch) -> int:
    """The hardware ceilings the GEMM kernels are measured against, measured
    on this box (inference-systems_amd/probes.py, csrc/probes.hip)."""
    import importlib

    P = importlib.import_module("inference_systems_amd.probes")
    P.load()
    out = {"probes": "MI355X ceilings on this box", "cus": P.CUS}
    # Clocks ramp under load: run the MFMA probe for ~0.3 s first.
    for _ in range(60):
        P.mfma_rate(torch, iters=512)
    out["launch_floor"] = P.launch_floor(torch)
    log(f"launch floor: {out['launch_floor']}")
    out["mfma_bf16_32x32x16"] = [P.mfma_rate(torch, workgroups=w, chains=c) for w in (P.CUS, 2 * P.CUS)
                                 for c in (4, 8)]
    log(f"mfma: {out['mfma_bf16_32x32x16']}")
    # The 16 x 16 x 32 instruction: a quarter of the flops per instruction,
    # so 4, 8 and 16 independent accumulators per wave.
    out["mfma_bf16_16x16x32"] = [P.mfma_rate(torch, workgroups=w, chains=c, shape="16x16x32")
                                 for w in (P.CUS, 2 * P.CUS) for c in (4, 8, 16)]
    log(f"mfma 16x16x32: {out['mfma_bf16_16x16x32']}")
    out["lds_read_b128"] = [P.lds_read(torch, workgroups=w) for w in (P.CUS, 2 * P.CUS)]
    log(f"lds reads: {out['lds_read_b128']}")
    out["lds_lane_groups"] = P.lds_lane_groups(torch)
    log(f"lds lane groups: {out['lds_lane_groups']}")
    # Copies from a window small enough for the vector L1 (16 KiB), for L2
    # (256 KiB and 4 MiB, read by every CU of an XCD), one workgroup per CU.
    # With three 1 KiB fragment reads per copied KiB (about a GEMM K-tile's
    # mix): whether the LDS serves the copies' writes and the reads at once.
    out["copy"] = [P.copy_rate(torch, mode, workgroups=P.CUS, inflight=f, window=win, reads=r)
                   for win in (16 << 10, 4 << 20) for mode in (0, 1, 2, 3) for f in (8, 16) for r in (0, 3)
                   if mode != 1 or r == 0]
    for r in out["copy"]:
        log(f"copy: {r}")
    # The C tiles of the bf16 prefill headline (2048 x 4096, 16.8 MB), written
    # by 256 workgroups at once as its epilogue does, one buffer and 16 in
    # rotation (past the Infinity Cache).
    out["write_c_tiles"] = [P.write_tiles(torch, nontemporal=nt, copies=c) for nt in (True, False) for c in (1, 16)]
    log(f"write C tiles: {out['write_c_tiles']}")
    decode_w = 6144 * 1024 * 2
    out["stream_read_decode_w"] = P.stream_read(torch, decode_w, math.ceil(2 * INFINITY_CACHE_BYTES / decode_w) + 1)
    log(f"stream read 12.6 MB: {out['stream_read_decode_w']}")
    head_w = 151936 * 1024 * 2
    out["stream_read_lm_head_w"] = P.stream_read(torch, head_w, 2, per_lane_list=(1, 4), reps_per_copy=2)
    log(f"stream read 311 MB: {out['stream_read_lm_head_w']}")
    print(json.dumps(out), flush=True)
    return 0


# Workloads with a single-call torch equivalent of the same output dtype:
# F.linear for W[N,K], torch.matmul for B[K,N] (the fp32-logit LM head has
# none: F.linear returns bf16).  Every input stays resident, ours included.
VENDOR_TUNED_CASES = (("bf16_prefill_2048x4096x1024", 2048), ("fp16_down_4096x1024x3584", 4096),
                      ("fp32_square_1024", 1024), ("bf16_decode_n6144_k1024", 1), ("bf16_decode_n6144_k1024", 8),
                      ("bf16_decode_n6144_k1024", 32))
VENDOR_TUNING_MS = 5          # TunableOp: time budget per candidate solution
VENDOR_TUNING_ITERATIONS = 20


def run_vendor_tuned(torch, L, W) -> int:
    """torch's GPU GEMM on each workload of VENDOR_TUNED_CASES with its
    default hipBLASLt / rocBLAS choice, then with the fastest solution
    TunableOp finds among all of them, beside the kernel selected here; each
    timed as 200 graph-replayed launches after a clock ramp."""
    import tempfile

    F = torch.nn.functional
    dev = torch.device("cuda:0")
    code = {torch.float32: L.F32, torch.float16: L.F16, torch.bfloat16: L.BF16}
    cases = []
    for name, m in VENDOR_TUNED_CASES:
        wl = W.WORKLOADS[name]
        a, b = W.make_inputs(name, m, device=dev)
        c = torch.empty((m, wl.n), dtype=wl.dtype_out, device=dev)
        ldb = wl.k if wl.b_layout == L.B_NK else wl.n
        raw = (a.data_ptr(), b.data_ptr(), c.data_ptr(), m, wl.n, wl.k, wl.k, ldb, wl.n, wl.b_layout,
               code[wl.dtype_in], code[wl.dtype_out])

        def ours(raw=raw):
            L.gemm_raw(*raw, torch.cuda.current_stream().cuda_stream)

        def vendor(a=a, b=b, nk=wl.b_layout == L.B_NK):
            if nk:
                F.linear(a, b)
            else:
                torch.matmul(a, b)
        cases.append((name, m, wl, ours, vendor))

    rows = []
    for name, m, wl, ours, vendor in cases:
        rows.append({"workload": name, "m": m, "n": wl.n, "k": wl.k, "flops": W.problem_flops(m, wl.n, wl.k),
                     "ours_us": median_graph_ms(torch, [ours] * 200) * 1e3,
                     "torch_default_us": median_graph_ms(torch, [vendor] * 200) * 1e3})
    T = torch.cuda.tunable
    results = Path(tempfile.mkdtemp()) / "tunableop_results.csv"
    T.set_filename(str(results))
    T.set_max_tuning_duration(VENDOR_TUNING_MS)
    T.set_max_tuning_iterations(VENDOR_TUNING_ITERATIONS)
    T.enable(True)
    T.tuning_enable(True)
    for (name, m, wl, ours, vendor), row in zip(cases, rows):
        vendor()                 # the search runs on the first call of a shape, outside any graph
        torch.cuda.synchronize()
        row["torch_tuned_us"] = median_graph_ms(torch, [vendor] * 200) * 1e3
    tuned = [list(r) for r in T.get_results()]
    T.tuning_enable(False)
    T.enable(False)
    for row in rows:
        # The entry whose parameter signature carries this GEMM's three sizes
        # (in TunableOp's m, n, k order, which follows the column-major call).
        want = sorted((row["m"], row["n"], row["k"]))
        for _, params, solution, _ in tuned:
            nums = [int(x) for x in re.findall(r"\d+", params)]
            if any(sorted(nums[i:i + 3]) == want for i in range(max(len(nums) - 2, 0))):
                row["torch_tuned_solution"] = solution
                break
        for key in ("ours_us", "torch_default_us", "torch_tuned_us"):
            row[key] = round(row[key], 3)
        row["ours_vs_tuned"] = round(row["torch_tuned_us"] / row["ours_us"], 3)
        tf = row.pop("flops")
        row["ours_TFLOP/s"] = round(tf / (row["ours_us"] * 1e-6) / 1e12, 2)
        log(f"{row['workload']} M={row['m']}: ours {row['ours_us']:.2f} us, torch default "
            f"{row['torch_default_us']:.2f} us, torch tuned {row['torch_tuned_us']:.2f} us "
            f"({row.get('torch_tuned_solution', '?')})")
    print(json.dumps({"vendor_tuned": "torch GPU GEMM, default and TunableOp-searched hipBLASLt / rocBLAS solution, "
                                      "against the selected kernel; inputs resident; 200 graph-replayed launches",
                      "tuning_ms_per_solution": VENDOR_TUNING_MS, "rows": rows, "tunableop_results": tuned}),
          flush=True)
    return 0


def _stability_cases(d: dict):
    """(case, ours_us, torch_us or None) of one default bench line."""
    yield (f"headline {d['config']['workload']}", d["ms_per_step"] * 1e3,
           d.get("vendor_torch_linear", {}).get("us"))
    if "headline_w_from_hbm" in d:
        yield "headline, W rotated from HBM", d["headline_w_from_hbm"]["us"], None
    for r in d.get("decode_bf16_n6144_k1024", []):
        yield f"bf16_decode_n6144_k1024 M={r['m']}", r["us"], r.get("torch_gpu_us")
    for r in d.get("other_workloads", []):
        yield f"{r['workload']} M={r['m']}", r["us"], r.get("torch_gpu_us")
    eo = d.get("eager_call_overhead")
    if eo:
        yield "eager call host time, nanovllm::gemm M=1", eo["rows"]["nanovllm::gemm"]["host_us"], \
            eo["rows"]["F.linear"]["host_us"]


def run_stability(runs: int) -> int:
    """The default bench (no CPU baseline) in `runs` fresh child processes;
    per case the mean, sample std, min and max of its microseconds, the same
    for torch's GPU GEMM where the bench times it, and torch / ours of the
    means.  This process imports neither torch nor the library."""
    import statistics
    import subprocess

    samples: dict = {}
    for i in range(runs):
        proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--no-cpu"], capture_output=True, text=True,
                              timeout=900)
        if proc.returncode != 0:
            print(proc.stderr[-2000:], file=sys.stderr)
            return proc.returncode
        d = json.loads(proc.stdout.strip().splitlines()[-1])
        for case, ours, vendor in _stability_cases(d):
            samples.setdefault(case, []).append((ours, vendor))
        log(f"stability run {i + 1}/{runs}: headline {d['ms_per_step'] * 1e3:.2f} us")

    def stats(xs):
        return {"mean": round(statistics.fmean(xs), 3), "std": round(statistics.stdev(xs), 3) if len(xs) > 1 else 0.0,
                "min": round(min(xs), 3), "max": round(max(xs), 3)}
    rows = []
    for case, vals in samples.items():
        ours = [v[0] for v in vals]
        row = {"case": case, "runs": len(ours), "us": stats(ours)}
        vend = [v[1] for v in vals if v[1] is not None]
        if len(vend) == len(ours):
            row["torch_us"] = stats(vend)
            row["torch_over_ours"] = round(statistics.fmean(vend) / statistics.fmean(ours), 3)
        rows.append(row)
        log(f"{case}: {row['us']['mean']:.2f} +- {row['us']['std']:.2f} us (min {row['us']['min']:.2f}, "
            f"max {row['us']['max']:.2f})" + (f"; torch {row['torch_us']['mean']:.2f} +- {row['torch_us']['std']:.2f}"
                                              f", torch/ours {row['torch_over_ours']:.3f}" if "torch_us" in row else ""))
    print(json.dumps({"stability": {"runs": runs, "command": "python3 bench.py --no-cpu, one fresh process per run",
                                    "rows": rows}}), flush=True)
    return 0


def run_data_patterns(torch, pkg) -> int:
    """Ours and torch's GPU GEMM on the same operands filled four ways:
    seeded random values (the bench's inputs), the same values with their
    mantissa bits cleared (sign and exponent kept), constants, and zeros.
    Graph replays of launches after a clock ramp; the same number of MFMAs,
    LDS accesses and bytes every time, only the bits differ.  torch's call
    is F.linear, or torch.mm(a, w.t(), out_dtype=torch.float32) for the
    LM head's fp32 logits."""
    L = pkg._lib
    W = pkg.workloads
    F = torch.nn.functional
    dev = torch.device("cuda:0")
    code = {torch.float16: L.F16, torch.bfloat16: L.BF16, torch.float32: L.F32}
    x = torch.randn(4096, 4096, device=dev, dtype=torch.bfloat16)
    for _ in range(200):
        x @ x
    rows = []
    for name, m, launches in (("bf16_prefill_2048x4096x1024", 2048, 100), ("fp16_down_4096x1024x3584", 4096, 100),
                              ("bf16_lm_head_n151936_k1024", 512, 20)):
        wl = W.WORKLOADS[name]
        a, w = W.make_inputs(name, m, device=dev)
        # sign and exponent bits, as the int16 view of the 16-bit pattern
        keep = -128 if wl.dtype_in == torch.bfloat16 else -1024   # 0xFF80 / 0xFC00
        fills = {
            "random": (a, w),
            "random, mantissa cleared": ((a.view(torch.int16) & keep).view(wl.dtype_in),
                                         (w.view(torch.int16) & keep).view(wl.dtype_in)),
            "constant": (torch.ones_like(a), torch.full_like(w, 0.02)),
            "zeros": (torch.zeros_like(a), torch.zeros_like(w)),
        }
        c = torch.empty(m, wl.n, dtype=wl.dtype_out, device=dev)
        if wl.dtype_out == torch.float32:
            torch_call = "torch.mm(a, w.t(), out_dtype=torch.float32)"
        else:
            torch_call = "F.linear(a, w)"
        for fill, (aa, ww) in fills.items():
            def ours(aa=aa, ww=ww):
                L.gemm_raw(aa.data_ptr(), ww.data_ptr(), c.data_ptr(), m, wl.n, wl.k, wl.k, wl.k, wl.n, L.B_NK,
                           code[wl.dtype_in], code[wl.dtype_out], torch.cuda.current_stream().cuda_stream)

            if wl.dtype_out == torch.float32:
                def theirs(aa=aa, ww=ww):
                    torch.mm(aa, ww.t(), out_dtype=torch.float32)
            else:
                def theirs(aa=aa, ww=ww):
                    F.linear(aa, ww)
            us = median_graph_ms(torch, [ours] * launches) * 1e3
            tus = median_graph_ms(torch, [theirs] * launches) * 1e3
            rows.append({"workload": name, "m": m, "inputs": fill, "us": round(us, 3), "torch_gpu_us": round(tus, 3),
                         "torch_call": torch_call})
            log(f"{name} M={m} {fill}: ours {us:.2f} us, torch {tus:.2f} us")
        del a, w, fills, c
    print(json.dumps({"data_patterns": rows}), flush=True)
    return 0


def run_counter_pair(torch, pkg, name: str, m, calls: int) -> int:
    """nanovllm::gemm and torch's equivalent on a workload's seeded inputs:
    one call of each compared, then two rounds of `calls` calls of ours and
    `calls` of torch's, for profiler counter passes that read both
    kernels on the same operands.  torch's call is F.linear (torch.matmul on
    B[K,N]), or torch.mm(a, w.t(), out_dtype=torch.float32) for fp32 outputs
    of 16-bit inputs."""
    W = pkg.workloads
    if name not in W.WORKLOADS:
        print(f"unknown workload {name!r}; choose from {sorted(W.WORKLOADS)}", file=sys.stderr)
        return 2
    wl = W.WORKLOADS[name]
    m = wl.ms[-1] if m is None else m
    a, b = W.make_inputs(name, m, device="cuda")
    nk = wl.b_layout == pkg._lib.B_NK
    op = torch.ops.nanovllm.gemm if nk else torch.ops.nanovllm.gemm_kn

    def ours():
        return op(a, b, wl.dtype_out)

    def theirs():
        if not nk:
            return torch.matmul(a, b)
        if wl.dtype_out == torch.float32 and wl.dtype_in != torch.float32:
            return torch.mm(a, b.t(), out_dtype=torch.float32)
        return torch.nn.functional.linear(a, b)

    diff = (ours().float() - theirs().float()).abs().max().item()
    log(f"{name} M={m}: max |ours - torch| = {diff:.3g}")
    for _ in range(2):
        for f in (ours, theirs):
            for _ in range(calls):
                f()
    torch.cuda.synchronize()
    print(json.dumps({"counter_pair": {"workload": name, "m": m, "calls": 1 + 2 * calls, "max_abs_diff": diff}}),
          flush=True)
    return 0


EAGER_CALLS = 2000
EAGER_TRIALS = 7


def eager_call_overhead(torch, pkg) -> dict:
    """Host microseconds per eager call on the decode shape (bf16, M = 1,
    W[6144, 1024]): `calls` launches issued back to back from Python, timed
    on the host clock before the final synchronize ("host_us", what the
    caller's thread spends per call) and after it ("wall_us").  The kernel
    takes ~3 us of GPU time, so both are host-bound.  Median of the trials.
    Under the op registration NANOVLLM_GEMM_OPS picks (kernels/gemm.py)."""
    import statistics
    import time

    F = torch.nn.functional
    G = sys.modules[pkg.__name__ + ".kernels.gemm"]
    L = pkg._lib
    dev = torch.device("cuda:0")
    a, w = pkg.workloads.make_inputs("bf16_decode_n6144_k1024", 1, device=dev)
    out = torch.empty(1, w.shape[0], dtype=torch.bfloat16, device=dev)
    raw = (a.data_ptr(), w.data_ptr(), out.data_ptr(), 1, w.shape[0], w.shape[1], w.shape[1], w.shape[1],
           w.shape[0], L.B_NK, L.BF16, L.BF16)
    calls = {
        "F.linear": lambda: F.linear(a, w),
        "nanovllm::gemm": lambda: torch.ops.nanovllm.gemm(a, w, None),
        "linear(backend=hip)": lambda: G.linear(a, w, None, backend="hip"),
        "C ABI through ctypes, output preallocated": lambda: L.gemm_raw(
            *raw, torch.cuda.current_stream().cuda_stream),
    }
    rows = {}
    for label, fn in calls.items():
        for _ in range(200):
            fn()
        torch.cuda.synchronize()
        host, wall = [], []
        for _ in range(EAGER_TRIALS):
            t0 = time.perf_counter()
            for _ in range(EAGER_CALLS):
                fn()
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            host.append((t1 - t0) / EAGER_CALLS * 1e6)
            wall.append((t2 - t0) / EAGER_CALLS * 1e6)
        rows[label] = {"host_us": round(statistics.median(host), 3), "wall_us": round(statistics.median(wall), 3)}
    return {"registration": G.REGISTRATION, "shape": "bf16 M=1 N=6144 K=1024, W[N,K]", "calls": EAGER_CALLS,
            "trials": EAGER_TRIALS, "rows": rows}


def eager_overhead_other_registration(registration: str) -> dict:
    """eager_call_overhead under another op registration, in a child process
    (an op name is registered once per process)."""
    import subprocess

    env = dict(os.environ, NANOVLLM_GEMM_OPS=registration)
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--eager-overhead"], env=env,
                          capture_output=True, text=True, timeout=600)
    if proc.returncode != 0:
        return {"registration": registration, "error": proc.stderr.strip()[-300:]}
    return json.loads(proc.stdout.strip().splitlines()[-1])["eager_call_overhead"]


# (N, K): q/k/v, down, merged GDN input projection, o_proj / GDN out_proj, a wide W
DECODE_SWEEP_SHAPES = ((6144, 1024), (1024, 3584), (8224, 1024), (1024, 2048), (16384, 1024))


def parse_shapes(text: str) -> tuple:
    """'151936x1024,6144x1024' -> ((151936, 1024), (6144, 1024))."""
    shapes = []
    for item in text.split(","):
        n, k = item.lower().split("x")
        shapes.append((int(n), int(k)))
        if shapes[-1][0] < 1 or shapes[-1][1] < 8 or shapes[-1][1] % 8:
            raise ValueError(f"bad W shape {item!r}: N >= 1 and K a positive multiple of 8")
    return tuple(shapes)


def run_decode_sweep(torch, L, shapes=DECODE_SWEEP_SHAPES) -> int:
    """Every configuration of the LDS-staged and the register-loading decode
    kernels (inference-systems_amd/csrc/decode_sweep.hip) on the bf16 decode
    shapes, W rotated past the Infinity Cache, graph replays as for the
    decode rows; each output checked against torch's fp32 product.  The
    selected kernel of the GEMM library is timed beside them."""
    import importlib

    P = importlib.import_module("inference_systems_amd.probes")
    cfgs = P.sweep_configs()
    out = {"decode_sweep": "bf16 in and out, W[N,K], W rotated past the Infinity Cache", "rows": []}
    gen = torch.Generator().manual_seed(2024)
    for n, k in shapes:
        w_cpu = (torch.randn(n, k, generator=gen) * 0.02).bfloat16()
        w0 = w_cpu.cuda()
        copies = max(2, math.ceil(2 * INFINITY_CACHE_BYTES / (n * k * 2)) + 1)
        ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        bs = [wt.t().contiguous() for wt in ws]    # the same matrices as B[K,N]
        for m in (1, 4, 8, 16, 32):
            a = torch.randn(m, k, generator=gen).bfloat16().cuda()
            ref = (a.float() @ w0.float().T)
            c = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
            kid = L.select(m, n, k, k, k, n, L.B_NK, L.BF16, L.BF16, True)

            def product(wt):
                args_ = (a.data_ptr(), wt.data_ptr(), c.data_ptr(), m, n, k, k, k, n, L.B_NK, L.BF16, L.BF16)
                return lambda: L.gemm_raw(*args_, torch.cuda.current_stream().cuda_stream)
            runs = [("selected " + L.kernel_name(kid), False, product)]
            for idx, name, max_m, kn in cfgs:
                if max_m >= m and max_m < 2 * max(m, 8):   # the configurations with the fewest rows of A that fit
                    runs.append((name, kn, lambda wt, idx=idx: P.sweep_launcher(torch, idx, a, wt, c)))
            for name, kn, make in runs:
                mats = bs if kn else ws
                c.zero_()
                make(mats[0])()
                torch.cuda.synchronize()
                err = float((c.float() - ref).abs().max())
                tol = float(ref.abs().max()) * 2 ** -7 + 1e-3
                t_ms = median_graph_ms(torch, [make(mats[i % copies]) for i in range(copies * 10)], trials=3)
                gbs = (n * k + m * k + m * n) * 2 / (t_ms * 1e-3) / 1e9
                row = {"n": n, "k": k, "m": m, "config": name, "us": round(t_ms * 1e3, 3), "GB/s": round(gbs, 1),
                       "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "max_abs_err": err, "ok": err <= tol}
                out["rows"].append(row)
                log(f"N={n} K={k} M={m:2d} {name:40s} {row['us']:7.2f} us  {gbs:6.0f} GB/s  "
                    f"err {err:.3g}{'' if row['ok'] else '  WRONG'}")
        del ws, bs, w0
        torch.cuda.empty_cache()
    print(json.dumps(out), flush=True)
    return 0 if all(r["ok"] for r in out["rows"]) else 1


def reference_inputs(torch, m: int, n: int, k: int):
    """A[M,K] and B[K,N] (fp32, CPU) from the reference's deterministic
    generators (gemm_bench.cu:296-305): multiples of 1/32 in [-15/32, 15/32]
    and [-14/32, 14/32], exact in fp16 and bf16."""
    ia = torch.arange(m * k, dtype=torch.int64)
    ib = torch.arange(k * n, dtype=torch.int64)
    a = (((ia * 17 + 3) % 31 - 15).to(torch.float32) * 0.03125).reshape(m, k)
    b = (((ib * 11 + 5) % 29 - 14).to(torch.float32) * 0.03125).reshape(k, n)
    return a, b


def reference_matrix(torch, L, W, dtypes=None, emit=print, rungs=True) -> list:
    """The reference's GEMM benchmark matrix on this GPU, one CSV row per
    (dtype, shape) as run_shape writes it (gemm_bench.cu:284-450,
    results/rtx3060_gemm_matrix.csv):

    * inputs from the reference's deterministic generators
      (gemm_bench.cu:296-305), A[M,K] and B[K,N] row-major, fp32 output;
      every product and partial sum of these inputs is exact in fp32, so
      the expected C is the same for any summation order;
    * the vendor column is torch's GPU GEMM (hipBLASLt / rocBLAS) with fp32
      output in place of cuBLAS, timed for comparison only;
    * every output is compared to the exact product (an fp64 GEMM, exact on
      these inputs) as compare does: max |error|, and pass if every error is
      within 5e-2 + 1e-2 |ref| and finite (gemm_bench.cu:225-250);
    * direct_*, staged_* and dispatch_* run on the reference's B[K,N]
      layout, as its columns do: mfma_direct, mfma_staged (B's k-rows copied
      as they lie, read back with the transposing LDS read) and the kernel
      the selection table picks for B[K,N]; the *_nk columns after the reference's run the same
      matrix transposed into the W[N,K] (nn.Linear) layout, where the decode
      kernels (gemv_decode, splitk_decode) also apply;
    * timing as benchmark_ms: 10 warm-up launches, repeats =
      clamp(2e10 / flops, 10, 200), median of 7 trials (gemm_bench.cu:371-379),
      each group of repeats replayed as one HIP graph (these kernels run for
      a few microseconds, less than a Python launch takes); the last column
      gives the selected kernel's time with plain launches from Python.
    """
    dev = torch.device("cuda:0")
    code = {torch.float16: L.F16, torch.bfloat16: L.BF16}
    cols = ["dtype", "label", "M", "N", "K", "repeats", "vendor_ms", "vendor_tflops", "direct_ms", "direct_tflops",
            "staged_ms", "staged_tflops", "vendor_max_abs", "direct_max_abs", "staged_max_abs", "dispatch",
            "dispatch_ms", "dispatch_tflops", "dispatch_max_abs", "dispatch_vs_vendor", "status",
            "dispatch_plain_launch_ms", "staged_nk_ms", "staged_nk_max_abs", "dispatch_nk", "dispatch_nk_ms",
            "dispatch_nk_max_abs", "dispatch_nk_plain_launch_ms"]
    emit(",".join(cols))
    rows = []
    for dt, dname in dtypes or ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        for label, m, n, k in W.QWEN35_SHAPES:
            a, b = reference_inputs(torch, m, n, k)
            a, b = a.to(dt).to(dev), b.to(dt).to(dev)
            w = b.t().contiguous()
            flops = 2.0 * m * n * k
            repeats = min(max(int(2.0e10 / max(flops, 1.0)), 10), 200)
            ref = torch.empty(m, n, dtype=torch.float32, device=dev)
            out = torch.empty(m, n, dtype=torch.float32, device=dev)

            expect = torch.mm(a.double(), b.double()).float()

            def vendor():
                torch.mm(a, b, out_dtype=torch.float32, out=ref)

            def ours(bt, layout, kernel=None):
                ldb = k if layout == L.B_NK else n
                args_ = (bt.data_ptr(), m, n, k, k, ldb, n, layout, code[dt], L.F32)

                def f():
                    L.gemm_raw(a.data_ptr(), args_[0], out.data_ptr(), *args_[1:],
                               torch.cuda.current_stream().cuda_stream, kernel=kernel)
                return f

            ok = True

            def run(f, dst):
                nonlocal ok
                t, t_plain = benchmark_ms(torch, f, 10, repeats)
                dst.fill_(float("nan"))
                f()
                torch.cuda.synchronize()
                err = (dst.double() - expect.double()).abs()
                good = bool(torch.isfinite(dst).all()) and bool((err <= 5e-2 + 1e-2 * expect.double().abs()).all())
                ok = ok and good
                return t, float(err.max()), t_plain

            try:
                vendor()
                vendor_ms, vendor_err, _ = run(vendor, ref)
            except RuntimeError:   # no fp32-output half GEMM in this torch build: comparison column left empty
                vendor_ms = vendor_err = float("nan")
            direct_ms = direct_err = staged_ms = staged_err = staged_nk_ms = staged_nk_err = float("nan")
            if rungs:   # the direct and staged rungs forced, beside the selected kernel
                direct_ms, direct_err, _ = run(ours(b, L.B_KN, L.KERNEL_MFMA_DIRECT), out)
                staged_ms, staged_err, _ = run(ours(b, L.B_KN, L.KERNEL_MFMA_STAGED), out)
                staged_nk_ms, staged_nk_err, _ = run(ours(w, L.B_NK, L.KERNEL_MFMA_STAGED), out)
            sel = L.select(m, n, k, k, n, n, L.B_KN, code[dt], L.F32)
            disp_ms, disp_err, disp_plain = run(ours(b, L.B_KN), out)
            sel_nk = L.select(m, n, k, k, k, n, L.B_NK, code[dt], L.F32)
            disp_nk_ms, disp_nk_err, disp_nk_plain = run(ours(w, L.B_NK), out)

            def tf(ms):
                return flops / (ms * 1e9)
            row = [dname, label, m, n, k, repeats, f"{vendor_ms:.6f}", f"{tf(vendor_ms):.6f}", f"{direct_ms:.6f}",
                   f"{tf(direct_ms):.6f}", f"{staged_ms:.6f}", f"{tf(staged_ms):.6f}", f"{vendor_err:.6f}",
                   f"{direct_err:.6f}",
                   f"{staged_err:.6f}", L.kernel_name(sel), f"{disp_ms:.6f}", f"{tf(disp_ms):.6f}",
                   f"{disp_err:.6f}", f"{vendor_ms / disp_ms:.6f}", "PASS" if ok else "FAIL", f"{disp_plain:.6f}",
                   f"{staged_nk_ms:.6f}", f"{staged_nk_err:.6f}", L.kernel_name(sel_nk), f"{disp_nk_ms:.6f}",
                   f"{disp_nk_err:.6f}", f"{disp_nk_plain:.6f}"]
            emit(",".join("NA" if x == "nan" else str(x) for x in row))
            rows.append(dict(zip(cols, row)))
            del a, b, w, ref, out, expect
            torch.cuda.empty_cache()
    return rows


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this GEMM path runs on one MI355X per process and has no "
              "multi-GPU mode (run with --gpus 1).", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2
    if args.stability:
        return run_stability(args.stability)

    import torch
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    L = pkg._lib
    L.load()                      # raises if the HIP library is not built
    W = pkg.workloads
    if args.probes:
        torch.cuda.set_device(0)
        return run_probes(torch)
    if args.decode_sweep:
        torch.cuda.set_device(0)
        shapes = parse_shapes(args.decode_sweep_shapes) if args.decode_sweep_shapes else DECODE_SWEEP_SHAPES
        return run_decode_sweep(torch, L, shapes)
    if args.vendor_tuned:
        torch.cuda.set_device(0)
        return run_vendor_tuned(torch, L, W)
    if args.counter_pair:
        torch.cuda.set_device(0)
        return run_counter_pair(torch, pkg, args.workload or W.HEADLINE, args.m, args.counter_pair)
    if args.data_patterns:
        torch.cuda.set_device(0)
        return run_data_patterns(torch, pkg)
    if args.eager_overhead:
        torch.cuda.set_device(0)
        print(json.dumps({"eager_call_overhead": eager_call_overhead(torch, pkg)}), flush=True)
        return 0
    if args.matrix:
        torch.cuda.set_device(0)
        rows = reference_matrix(torch, L, W, emit=lambda line: print(line, flush=True))
        return 0 if all(r["status"] == "PASS" for r in rows) else 1
    K_ops = pkg.kernels
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    code = {torch.float32: L.F32, torch.float16: L.F16, torch.bfloat16: L.BF16}
    dname = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}

    def launcher(a, b, c, m, n, k, layout, din, dout):
        ldb = k if layout == L.B_NK else n
        args_ = (a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, k, ldb, n, layout, code[din], code[dout])

        def f():
            L.gemm_raw(*args_, torch.cuda.current_stream().cuda_stream)
        return f

    # ---------------------------------------------------------------- headline
    name = args.workload or W.HEADLINE
    if name not in W.WORKLOADS:
        print(f"unknown workload {name!r}; choose from {sorted(W.WORKLOADS)}", file=sys.stderr)
        return 2
    wl = W.WORKLOADS[name]
    m = args.m if args.m is not None else wl.ms[-1]
    n, k = wl.n, wl.k
    a, w = W.make_inputs(name, m, device=dev)
    out = torch.empty(m, n, dtype=wl.dtype_out, device=dev)
    ldb_h = k if wl.b_layout == L.B_NK else n
    kid = L.select(m, n, k, k, ldb_h, n, wl.b_layout, code[wl.dtype_in], code[wl.dtype_out], True)
    kernel = L.kernel_name(kid)
    flops = W.problem_flops(m, n, k)
    # Bandwidth-bound problems rotate W over more than twice the Infinity
    # Cache so every launch streams W from HBM.
    copies = 1
    if wl.bound == "hbm":
        w_bytes = w.numel() * w.element_size()
        copies = max(2, math.ceil(2 * INFINITY_CACHE_BYTES / w_bytes) + 1)
    ws_h = [w] + [w.clone() for _ in range(copies - 1)]
    launches = [launcher(a, ws_h[i % copies], out, m, n, k, wl.b_layout, wl.dtype_in, wl.dtype_out)
                for i in range(copies)]
    log(f"headline {name} M={m}: kernel {kernel}, W buffers {copies}, warmup {args.warmup}, steps {args.steps}")
    # Graphs are captured first: capture is host work that leaves the GPU
    # idle, and an idle MI355X drops its clocks.
    steps = [launches[i % copies] for i in range(args.steps)]
    timer = GraphTimer(torch, steps)
    warm_graph = GraphTimer(torch, steps[:args.warmup]) if args.warmup > 0 and wl.bound != "mfma" else None
    # Device warm-up: MI355X clocks ramp over the first ~0.1-0.2 s of load
    # (the same kernel measured 10% slower in its first 100 launches), so run
    # the kernel for DEVICE_WARMUP_S right before the warm-up steps.  Untimed.
    ramp = GraphTimer(torch, [launches[i % copies] for i in range(200)])
    t_ramp = 0.0
    while t_ramp < DEVICE_WARMUP_S * 1e3:
        t_ramp += ramp.time_ms()
    del ramp
    if wl.bound == "mfma":
        # Kernels of ~10 us and more: K launches issued back to back on the
        # stream and timed with HIP events, the pattern of the reference's
        # benchmark_ms (gemm_bench.cu:198-223); the graph replay of the same
        # K launches is reported beside it.
        for f in steps[:args.warmup]:
            f()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for f in steps:
            f()
        end.record()
        torch.cuda.synchronize()
        elapsed_ms = start.elapsed_time(end)
        other_ms = timer.time_ms() / args.steps
        timing = "K launches back to back on one stream, HIP events; graph_ms_per_step: the same K in one HIP graph"
    else:
        # Short, bandwidth-bound kernels: the K launches replayed as one HIP
        # graph, so host launch gaps are excluded; plain stream launches
        # reported beside.
        if warm_graph is not None:
            warm_graph.time_ms()
        torch.cuda.synchronize()
        elapsed_ms = timer.time_ms()
        torch.cuda.synchronize()
        other_ms = median_plain_ms(torch, steps[:200], trials=3)
        timing = "K launches back to back in one HIP graph, HIP events; plain_launch_ms_per_step: stream launches"
    ms_per_step = elapsed_ms / args.steps
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    peak = PEAK_MFMA_TFLOPS[dname[wl.dtype_in]]
    byts = W.problem_bytes(m, n, k, wl.dtype_in, wl.dtype_out)
    gbs = byts / (ms_per_step * 1e-3) / 1e9
    log(f"  {ms_per_step * 1e3:.2f} us/step  {tflops:.1f} TFLOP/s  {100 * tflops / peak:.1f}% of {peak} TFLOP/s  "
        f"{gbs:.0f} GB/s  {100 * gbs / PEAK_HBM_GBS:.1f}% of HBM  ({timing.split(';')[0]}; "
        f"{'graph' if wl.bound == 'mfma' else 'plain'}: {other_ms * 1e3:.2f} us/step)")
    if wl.bound == "hbm":
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(tflops, 3), "peak": peak, "unit": "TFLOP/s",
                "frac": round(tflops / peak, 4)}
    roof.update({"traffic": read_traffic() if name == W.HEADLINE else None,
                 "algorithmic_flops_per_launch": flops, "algorithmic_bytes_per_launch": byts})

    result = {
        "metric": "TFLOP/s & % MFMA peak (prefill GEMM); HBM GB/s & % peak (decode M<=32)",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        ("graph_ms_per_step" if wl.bound == "mfma" else "plain_launch_ms_per_step"): round(other_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname[wl.dtype_in],
        "data": "synthetic (seeded random activations and weights, rounded to the input dtype)",
        "config": {"workload": name, "m": m, "n": n, "k": k,
                   "b_layout": "W[N,K]" if wl.b_layout == L.B_NK else "B[K,N]",
                   "out_dtype": dname[wl.dtype_out], "kernel": kernel,
                   "w_buffers": copies, "device_warmup_s": DEVICE_WARMUP_S,
                   "timing": timing},
        "roofline": roof,
    }

    extras = {}
    # ----------------------------------------- headline with W read cold
    # The headline reuses one W, which stays in the 256 MB Infinity Cache
    # across launches; a model's prefill reads each layer's W once.  Here W
    # rotates over enough copies that every launch reads it from HBM (A and
    # C stay one buffer each), timed the same way.
    if not args.no_extras and wl.bound == "mfma":
        r_copies = math.ceil(2 * INFINITY_CACHE_BYTES / (w.numel() * w.element_size())) + 1
        r_ws = [w] + [w.clone() for _ in range(r_copies - 1)]
        r_steps = [launcher(a, r_ws[i % r_copies], out, m, n, k, wl.b_layout, wl.dtype_in, wl.dtype_out)
                   for i in range(r_copies * 4)]
        for f in r_steps:
            f()
        torch.cuda.synchronize()
        r_start, r_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        r_start.record()
        for f in r_steps:
            f()
        r_end.record()
        torch.cuda.synchronize()
        r_ms = r_start.elapsed_time(r_end) / len(r_steps)
        extras["headline_w_from_hbm"] = {"us": round(r_ms * 1e3, 3), "TFLOP/s": round(flops / (r_ms * 1e-3) / 1e12, 2),
                                         "frac_mfma": round(flops / (r_ms * 1e-3) / 1e12 / peak, 4),
                                         "w_buffers": r_copies, "launches": len(r_steps)}
        log(f"headline with W rotated over {r_copies} buffers: {r_ms * 1e3:.2f} us/step")
        del r_ws, r_steps

    # ------------------------------------------------------------ decode rows
    if not args.no_extras:
        dname_ = "bf16_decode_n6144_k1024"
        dw = W.WORKLOADS[dname_]
        w_bytes = dw.n * dw.k * 2
        copies = max(2, math.ceil(2 * INFINITY_CACHE_BYTES / w_bytes) + 1)
        _, w0 = W.make_inputs(dname_, 1, device=dev)
        ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        rows = []
        for dm in dw.ms:
            a_d, _ = W.make_inputs(dname_, dm, device=dev)
            o_d = torch.empty(dm, dw.n, dtype=dw.dtype_out, device=dev)
            launches = [launcher(a_d, ws[i % copies], o_d, dm, dw.n, dw.k, L.B_NK, dw.dtype_in, dw.dtype_out)
                        for i in range(copies * 10)]
            t_ms = median_graph_ms(torch, launches)
            t_plain = median_plain_ms(torch, launches)
            # torch's GPU GEMM (F.linear) over the same W rotation
            t_torch = median_graph_ms(torch, [(lambda bb=ws[i % copies], aa=a_d: torch.nn.functional.linear(aa, bb))
                                              for i in range(copies * 10)])
            byts = W.problem_bytes(dm, dw.n, dw.k, dw.dtype_in, dw.dtype_out)
            gbs = byts / (t_ms * 1e-3) / 1e9
            kd = L.kernel_name(L.select(dm, dw.n, dw.k, dw.k, dw.k, dw.n, L.B_NK, L.BF16, L.BF16, True))
            rows.append({"m": dm, "us": round(t_ms * 1e3, 3), "GB/s": round(gbs, 1),
                         "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "kernel": kd, "w_buffers": copies,
                         "plain_launch_us": round(t_plain * 1e3, 3), "torch_gpu_us": round(t_torch * 1e3, 3),
                         "torch_gpu_call": "F.linear(a, w)"})
            log(f"decode M={dm:2d}: {t_ms * 1e3:.2f} us  {gbs:.0f} GB/s  {100 * gbs / PEAK_HBM_GBS:.1f}% of HBM ({kd}); "
                f"plain stream launches {t_plain * 1e3:.2f} us; torch F.linear {t_torch * 1e3:.2f} us")
        extras["decode_bf16_n6144_k1024"] = rows
        del ws

        # ------------------------------------------------ other workloads
        other = []
        for oname in ("fp32_square_1024", "fp16_down_4096x1024x3584", "bf16_lm_head_n151936_k1024"):
            ow = W.WORKLOADS[oname]
            for om in ow.ms:
                a_o, b_o = W.make_inputs(oname, om, device=dev)
                o_o = torch.empty(om, ow.n, dtype=ow.dtype_out, device=dev)
                b_bytes = b_o.numel() * b_o.element_size()
                nbuf = 2 if ow.bound == "hbm" else 1
                bs = [b_o] + [b_o.clone() for _ in range(nbuf - 1)]
                reps = 20 if b_bytes > 2 ** 27 else 100
                launches = [launcher(a_o, bs[i % nbuf], o_o, om, ow.n, ow.k, ow.b_layout, ow.dtype_in,
                                     ow.dtype_out) for i in range(reps)]
                t_ms = median_graph_ms(torch, launches, trials=3)
                # torch's GPU GEMM on the same operands (the same W rotation):
                # F.linear on W[N,K], torch.matmul on B[K,N], and for fp32
                # logits from bf16 torch.mm(a, w.t(), out_dtype=torch.float32).
                if ow.b_layout != L.B_NK:
                    v_call, v_fn = "torch.matmul(a, b)", (lambda aa, bb: torch.matmul(aa, bb))
                elif ow.dtype_out != ow.dtype_in:
                    v_call = "torch.mm(a, w.t(), out_dtype=torch.float32)"
                    v_fn = (lambda aa, bb: torch.mm(aa, bb.t(), out_dtype=torch.float32))
                else:
                    v_call, v_fn = "F.linear(a, w)", (lambda aa, bb: torch.nn.functional.linear(aa, bb))
                try:
                    v_ms = median_graph_ms(torch, [(lambda bb=bs[i % nbuf], aa=a_o: v_fn(aa, bb))
                                                   for i in range(reps)], trials=3)
                except Exception as exc:  # comparison only; never fails the bench
                    v_ms, v_call = float("nan"), f"{v_call}: {str(exc)[:120]}"
                fl = W.problem_flops(om, ow.n, ow.k)
                byts = W.problem_bytes(om, ow.n, ow.k, ow.dtype_in, ow.dtype_out)
                tf = fl / (t_ms * 1e-3) / 1e12
                gbs = byts / (t_ms * 1e-3) / 1e9
                pk = PEAK_MFMA_TFLOPS[dname[ow.dtype_in]]
                ldb = ow.k if ow.b_layout == L.B_NK else ow.n
                ko = L.kernel_name(L.select(om, ow.n, ow.k, ow.k, ldb, ow.n, ow.b_layout, code[ow.dtype_in],
                                            code[ow.dtype_out], True))
                other.append({"workload": oname, "m": om, "us": round(t_ms * 1e3, 3), "TFLOP/s": round(tf, 2),
                              "frac_mfma": round(tf / pk, 4), "GB/s": round(gbs, 1),
                              "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "kernel": ko,
                              "torch_gpu_us": None if math.isnan(v_ms) else round(v_ms * 1e3, 3),
                              "torch_gpu_call": v_call})
                log(f"{oname} M={om}: {t_ms * 1e3:.1f} us  {tf:.1f} TFLOP/s ({100 * tf / pk:.1f}%)  "
                    f"{gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}%)  [{ko}]; torch {v_ms * 1e3:.1f} us ({v_call})")
                del bs, a_o, b_o, o_o
        extras["other_workloads"] = other

        # ----------------------- merged gated-delta-net input projection
        # One N = 8224 GEMM (6144 + 2048 + 16 + 16 rows of W) against the four
        # launches of gated_delta_net.py:192-195, W streamed from HBM.
        g_gen = torch.Generator().manual_seed(1006)
        g_rows = (6144, 2048, 16, 16)
        g_w = (torch.randn(sum(g_rows), 1024, generator=g_gen) * 0.02).bfloat16().to(dev)
        g_copies = max(2, math.ceil(2 * INFINITY_CACHE_BYTES / (g_w.numel() * 2)) + 1)
        g_ws = [g_w] + [g_w.clone() for _ in range(g_copies - 1)]
        g_rows_out = []
        for gm in (1, 32):
            g_a = torch.randn(gm, 1024, generator=g_gen).bfloat16().to(dev)
            g_out = torch.empty(gm, sum(g_rows), dtype=torch.bfloat16, device=dev)
            merged = [launcher(g_a, g_ws[i % g_copies], g_out, gm, sum(g_rows), 1024, L.B_NK, torch.bfloat16,
                               torch.bfloat16) for i in range(g_copies * 2)]
            g_parts = [torch.empty(gm, rows, dtype=torch.bfloat16, device=dev) for rows in g_rows]
            separate = []
            for i in range(g_copies * 2):
                off = 0
                for rows, part in zip(g_rows, g_parts):
                    separate.append(launcher(g_a, g_ws[i % g_copies][off:off + rows], part, gm, rows, 1024,
                                             L.B_NK, torch.bfloat16, torch.bfloat16))
                    off += rows
            t_one = median_graph_ms(torch, merged)
            t_four = median_graph_ms(torch, separate) * len(g_rows)   # per step of four launches

            def merged_contiguous(f):
                def g():
                    f()
                    for part in g_out.split(g_rows, dim=-1):
                        part.contiguous()   # the copies GdnInputProjection.forward(contiguous=True) avoids
                return g
            t_cont = median_graph_ms(torch, [merged_contiguous(f) for f in merged])
            g_rows_out.append({"m": gm, "merged_us": round(t_one * 1e3, 3), "four_launches_us": round(t_four * 1e3, 3),
                               "speedup": round(t_four / t_one, 3),
                               "merged_with_contiguous_parts_us": round(t_cont * 1e3, 3)})
            log(f"gdn input projection M={gm}: merged {t_one * 1e3:.2f} us (with contiguous parts "
                f"{t_cont * 1e3:.2f} us), four launches {t_four * 1e3:.2f} us")
        extras["gdn_input_projection_bf16_k1024"] = g_rows_out
        del g_ws, g_w

        # --------------- fused MLP gate/up projection + SiLU-and-mul
        # One launch of the fused kernel against the reference's composition
        # (gate_up GEMM writing [M, 7168], then F.silu(gate) * up on the GPU).
        F_ = torch.nn.functional
        inter = 3584
        s_gen = torch.Generator().manual_seed(1007)
        s_w = (torch.randn(2 * inter, 1024, generator=s_gen) * 0.02).bfloat16().to(dev)
        s_rows = []
        for sm in (1, 32, 2048):
            s_copies = max(2, math.ceil(2 * INFINITY_CACHE_BYTES / (s_w.numel() * 2)) + 1) if sm <= 32 else 1
            s_ws = [s_w] + [s_w.clone() for _ in range(s_copies - 1)]
            s_a = torch.randn(sm, 1024, generator=s_gen).bfloat16().to(dev)
            s_out = torch.empty(sm, inter, dtype=torch.bfloat16, device=dev)
            s_gu = torch.empty(sm, 2 * inter, dtype=torch.bfloat16, device=dev)

            def fused(wt, s_a=s_a, s_out=s_out, sm=sm):
                args_ = (s_a.data_ptr(), wt.data_ptr(), s_out.data_ptr(), sm, inter, 1024, 1024, 1024, inter,
                         L.BF16, L.BF16)

                def f():
                    L.silu_mul_raw(*args_, torch.cuda.current_stream().cuda_stream)
                return f

            def unfused(wt, s_a=s_a, s_gu=s_gu, sm=sm):
                gemm = launcher(s_a, wt, s_gu, sm, 2 * inter, 1024, L.B_NK, torch.bfloat16, torch.bfloat16)

                def f():
                    gemm()
                    gate, up = s_gu.chunk(2, -1)
                    F_.silu(gate) * up
                return f
            reps = s_copies * 4 if sm <= 32 else 40
            t_f = median_graph_ms(torch, [fused(s_ws[i % s_copies]) for i in range(reps)])
            t_u = median_graph_ms(torch, [unfused(s_ws[i % s_copies]) for i in range(reps)])
            kf = L.kernel_name(L.silu_mul_select(sm, inter, 1024, 1024, 1024, inter, L.BF16, L.BF16, True))
            s_rows.append({"m": sm, "fused_us": round(t_f * 1e3, 3), "unfused_us": round(t_u * 1e3, 3),
                           "speedup": round(t_u / t_f, 3), "kernel": kf})
            log(f"mlp gate_up+SiLU-and-mul M={sm}: fused {t_f * 1e3:.2f} us ({kf}), "
                f"GEMM + torch SiluAndMul {t_u * 1e3:.2f} us")
            del s_ws
        extras["mlp_gate_up_silu_mul_bf16_n3584_k1024"] = s_rows
        del s_w

        # ----------------------------- greedy LM head (argmax, no logits)
        # Against the reference's path: bf16 logits [M, 151936] from the GEMM
        # (F.linear in the model dtype, embed_head.py:61), then
        # logits.float().argmax(dim=-1) (sampler.py:15, 21) on the GPU.  The
        # fused head ranks the same bf16-rounded logits.
        lw = W.WORKLOADS["bf16_lm_head_n151936_k1024"]
        _, l_w0 = W.make_inputs("bf16_lm_head_n151936_k1024", 1, device=dev)
        l_ws = [l_w0, l_w0.clone()]
        l_rows = []
        for lm in (1, 32):
            l_a, _ = W.make_inputs("bf16_lm_head_n151936_k1024", lm, device=dev)
            l_tok = torch.empty(lm, dtype=torch.int64, device=dev)
            l_val = torch.empty(lm, dtype=torch.float32, device=dev)
            l_need = L.argmax_workspace_bytes(lm, lw.n, lw.k, lw.k, lw.k, L.BF16)
            l_ws_buf = torch.empty(l_need, dtype=torch.uint8, device=dev)
            l_logits = torch.empty(lm, lw.n, dtype=torch.bfloat16, device=dev)

            def greedy(wt, l_a=l_a, l_tok=l_tok, l_val=l_val, l_ws_buf=l_ws_buf, lm=lm, l_need=l_need):
                args_ = (l_a.data_ptr(), wt.data_ptr(), l_tok.data_ptr(), l_val.data_ptr(), lm, lw.n, lw.k, lw.k,
                         lw.k, L.BF16, L.BF16, l_ws_buf.data_ptr(), l_need)

                def f():
                    L.argmax_raw(*args_, torch.cuda.current_stream().cuda_stream)
                return f

            def logits_then_argmax(wt, l_a=l_a, l_logits=l_logits, lm=lm):
                gemm = launcher(l_a, wt, l_logits, lm, lw.n, lw.k, L.B_NK, torch.bfloat16, torch.bfloat16)

                def f():
                    gemm()
                    l_logits.float().argmax(dim=-1)
                return f
            t_g = median_graph_ms(torch, [greedy(l_ws[i % 2]) for i in range(20)], trials=3)
            t_l = median_graph_ms(torch, [logits_then_argmax(l_ws[i % 2]) for i in range(20)], trials=3)
            l_rows.append({"m": lm, "greedy_us": round(t_g * 1e3, 3), "logits_then_argmax_us": round(t_l * 1e3, 3),
                           "speedup": round(t_l / t_g, 3)})
            log(f"lm head greedy M={lm}: fused {t_g * 1e3:.1f} us, bf16 logits + torch argmax {t_l * 1e3:.1f} us")
        extras["lm_head_greedy_bf16_n151936_k1024"] = l_rows

        # ----------------------------- sampled LM head (Sampler, no logits)
        # Every row sampled at temperature 0.8, against the reference's path:
        # bf16 logits from the GEMM, then Sampler.forward (sampler.py:8-21:
        # softmax, exponential draws, divide, argmax; eager here, the
        # reference wraps it in torch.compile).
        p_rows = []
        for lm in (1, 32):
            l_a, _ = W.make_inputs("bf16_lm_head_n151936_k1024", lm, device=dev)
            p_tok = torch.empty(lm, dtype=torch.int64, device=dev)
            p_val = torch.empty(lm, dtype=torch.float32, device=dev)
            p_temp = torch.full((lm,), 0.8, dtype=torch.float32, device=dev)
            p_need = L.argmax_workspace_bytes(lm, lw.n, lw.k, lw.k, lw.k, L.BF16)
            p_ws_buf = torch.empty(p_need, dtype=torch.uint8, device=dev)
            p_logits = torch.empty(lm, lw.n, dtype=torch.bfloat16, device=dev)

            def sampled(wt, step, l_a=l_a, p_tok=p_tok, p_val=p_val, p_temp=p_temp, p_ws_buf=p_ws_buf, lm=lm,
                        p_need=p_need):
                def f():
                    L.sample_raw(l_a.data_ptr(), wt.data_ptr(), p_temp.data_ptr(), 1234, step, p_tok.data_ptr(),
                                 p_val.data_ptr(), lm, lw.n, lw.k, lw.k, lw.k, L.BF16, L.BF16, p_ws_buf.data_ptr(),
                                 p_need,
                                 torch.cuda.current_stream().cuda_stream)
                return f

            def logits_then_sampler(wt, l_a=l_a, p_logits=p_logits, p_temp=p_temp, lm=lm):
                gemm = launcher(l_a, wt, p_logits, lm, lw.n, lw.k, L.B_NK, torch.bfloat16, torch.bfloat16)

                def f():
                    gemm()
                    K_ops.torch_sampler(p_logits, p_temp)
                return f
            t_s = median_graph_ms(torch, [sampled(l_ws[i % 2], i) for i in range(20)], trials=3)
            t_r = median_graph_ms(torch, [logits_then_sampler(l_ws[i % 2]) for i in range(20)], trials=3)
            p_rows.append({"m": lm, "sampled_us": round(t_s * 1e3, 3),
                           "logits_then_sampler_us": round(t_r * 1e3, 3), "speedup": round(t_r / t_s, 3)})
            log(f"lm head sampled (T=0.8) M={lm}: fused {t_s * 1e3:.1f} us, "
                f"bf16 logits + eager torch Sampler {t_r * 1e3:.1f} us")
        extras["lm_head_sampled_bf16_n151936_k1024"] = p_rows
        del l_ws, l_w0

        # ------------------- gated-attention output gate fused before o_proj
        # Against the reference's path: `output * torch.sigmoid(gate)` on the
        # GPU (two element-type ops, qwen3_5.py:95), then the o_proj GEMM.
        PK = pkg.kernels
        heads, hd, o_n = 8, 256, 1024
        o_k = heads * hd
        o_gen = torch.Generator().manual_seed(1011)
        o_w = (torch.randn(o_n, o_k, generator=o_gen) * 0.02).bfloat16().to(dev)
        o_rows = []
        for om in (1, 8, 32, 2048):
            o_copies = max(2, math.ceil(2 * INFINITY_CACHE_BYTES / (o_w.numel() * 2)) + 1) if om <= 32 else 1
            o_ws = [o_w] + [o_w.clone() for _ in range(o_copies - 1)]
            o_a = torch.randn(om, heads, hd, generator=o_gen).bfloat16().to(dev)
            o_q = (torch.randn(om, heads, 2 * hd, generator=o_gen) * 2).bfloat16().to(dev)
            o_gate = o_q.chunk(2, -1)[1]
            o_out = torch.empty(om, o_n, dtype=torch.bfloat16, device=dev)
            o_need = L.gated_workspace_bytes(om, o_k, hd, L.BF16)
            o_buf = torch.empty(o_need, dtype=torch.uint8, device=dev)
            o_gated = torch.empty(om, o_k, dtype=torch.bfloat16, device=dev)

            def gated(wt, o_a=o_a, o_gate=o_gate, o_out=o_out, o_buf=o_buf, om=om, o_need=o_need):
                args_ = (o_a.data_ptr(), o_gate.data_ptr(), wt.data_ptr(), o_out.data_ptr(), om, o_n, o_k, o_k,
                         o_gate.stride(0), hd, o_gate.stride(1), o_k, o_n, L.BF16, L.BF16, o_buf.data_ptr(), o_need)

                def f():
                    L.gated_raw(*args_, torch.cuda.current_stream().cuda_stream)
                return f

            def gate_then_gemm(wt, o_a=o_a, o_gate=o_gate, o_gated=o_gated, o_out=o_out, om=om):
                gemm = launcher(o_gated, wt, o_out, om, o_n, o_k, L.B_NK, torch.bfloat16, torch.bfloat16)

                def f():
                    torch.mul(o_a, torch.sigmoid(o_gate), out=o_gated.view(om, heads, hd))
                    gemm()
                return f
            reps = min(o_copies * 2, 400) if om <= 32 else 40
            t_f = median_graph_ms(torch, [gated(o_ws[i % o_copies]) for i in range(reps)])
            t_u = median_graph_ms(torch, [gate_then_gemm(o_ws[i % o_copies]) for i in range(reps)])
            o_rows.append({"m": om, "fused_us": round(t_f * 1e3, 3), "torch_gate_then_gemm_us": round(t_u * 1e3, 3),
                           "speedup": round(t_u / t_f, 3), "fused_in_gemm": om <= 8})
            log(f"o_proj with output gate M={om}: fused {t_f * 1e3:.2f} us, "
                f"torch sigmoid gate + GEMM {t_u * 1e3:.2f} us")
            del o_ws
        extras["attn_o_proj_gated_bf16_n1024_k2048"] = o_rows
        del o_w

        # ----------- residual add + RMSNorm fused before the next projection
        # Against the reference's path: Qwen3_5RMSNorm(h, residual) in eager
        # torch (layernorm.py:131-142), then the GEMM (for the MLP block, the
        # fused gate_up + SiLU GEMM).
        n_rows = []
        n_gen = torch.Generator().manual_seed(1013)
        for label, n_out, silu in (("gdn_in_proj_n8224", 8224, False), ("mlp_gate_up_silu_n3584", 3584, True)):
            n_w = (torch.randn((2 if silu else 1) * n_out, 1024, generator=n_gen) * 0.02).bfloat16().to(dev)
            n_nw = (torch.randn(1024, generator=n_gen) * 0.1).bfloat16().to(dev)
            for nm in (1, 32, 2048):
                n_copies = max(2, math.ceil(2 * INFINITY_CACHE_BYTES / (n_w.numel() * 2)) + 1) if nm <= 32 else 1
                n_ws = [n_w] + [n_w.clone() for _ in range(n_copies - 1)]
                n_h = torch.randn(nm, 1024, generator=n_gen).bfloat16().to(dev)
                n_r = torch.randn(nm, 1024, generator=n_gen).bfloat16().to(dev)
                n_out_t = torch.empty(nm, n_out, dtype=torch.bfloat16, device=dev)
                n_res = torch.empty(nm, 1024, dtype=torch.bfloat16, device=dev)
                n_need = L.add_rmsnorm_workspace_bytes(nm, 1024, L.BF16)
                n_buf = torch.empty(n_need, dtype=torch.uint8, device=dev)

                def fused_norm(wt, n_h=n_h, n_r=n_r, n_out_t=n_out_t, n_res=n_res, n_buf=n_buf, nm=nm,
                               n_need=n_need, n_nw=n_nw, n_out=n_out, silu=silu):
                    args_ = (n_h.data_ptr(), n_r.data_ptr(), n_nw.data_ptr(), 1e-6, wt.data_ptr(), n_out_t.data_ptr(),
                             n_res.data_ptr(), nm, n_out, 1024, 1024, 1024, 1024, n_out, 1024, silu, L.BF16, L.BF16,
                             n_buf.data_ptr(), n_need)

                    def f():
                        L.add_rmsnorm_raw(*args_, torch.cuda.current_stream().cuda_stream)
                    return f

                def norm_then_gemm(wt, n_h=n_h, n_r=n_r, n_out_t=n_out_t, nm=nm, n_nw=n_nw, n_out=n_out, silu=silu):
                    def f():
                        normed, _ = PK.torch_add_rmsnorm(n_h, n_r, n_nw, 1e-6)
                        if silu:
                            L.silu_mul_raw(normed.data_ptr(), wt.data_ptr(), n_out_t.data_ptr(), nm, n_out, 1024,
                                           1024, 1024, n_out, L.BF16, L.BF16, torch.cuda.current_stream().cuda_stream)
                        else:
                            L.gemm_raw(normed.data_ptr(), wt.data_ptr(), n_out_t.data_ptr(), nm, n_out, 1024, 1024,
                                       1024, n_out, L.B_NK, L.BF16, L.BF16, torch.cuda.current_stream().cuda_stream)
                    return f
                reps = min(n_copies * 2, 200) if nm <= 32 else 20
                t_f = median_graph_ms(torch, [fused_norm(n_ws[i % n_copies]) for i in range(reps)])
                t_u = median_graph_ms(torch, [norm_then_gemm(n_ws[i % n_copies]) for i in range(reps)])
                n_rows.append({"block": label, "m": nm, "fused_us": round(t_f * 1e3, 3),
                               "torch_norm_then_gemm_us": round(t_u * 1e3, 3), "speedup": round(t_u / t_f, 3),
                               "fused_in_gemm": nm <= 32})
                log(f"add+RMSNorm before {label} M={nm}: fused {t_f * 1e3:.2f} us, "
                    f"torch Qwen3_5RMSNorm + GEMM {t_u * 1e3:.2f} us")
                del n_ws
            del n_w
        extras["add_rmsnorm_before_projection_bf16_k1024"] = n_rows

    # --------------------------- the reference's shape matrix, bf16 rows
    if not args.no_extras and name == W.HEADLINE:
        mrows = reference_matrix(torch, L, W, dtypes=((torch.bfloat16, "bf16"),), emit=lambda line: None,
                                 rungs=False)
        extras["reference_shape_matrix_bf16"] = [
            {"shape": r["label"], "m": r["M"], "n": r["N"], "k": r["K"], "kernel_b_kn": r["dispatch"],
             "us_b_kn": round(float(r["dispatch_ms"]) * 1e3, 3), "kernel_w_nk": r["dispatch_nk"],
             "us_w_nk": round(float(r["dispatch_nk_ms"]) * 1e3, 3),
             "torch_gpu_gemm_us": None if r["vendor_ms"] == "nan" else round(float(r["vendor_ms"]) * 1e3, 3),
             "exact": r["status"] == "PASS"} for r in mrows]
        log("reference shape matrix (bf16, fp32 out; B[K,N] / W[N,K]): " + ", ".join(
            f"{r['label']} {float(r['dispatch_ms']) * 1e3:.2f} / {float(r['dispatch_nk_ms']) * 1e3:.2f} us"
            for r in mrows))

    # ------------------------------------- host cost of one eager call
    if not args.no_extras:
        eo = eager_call_overhead(torch, pkg)
        other_reg = [r for r in sys.modules[pkg.__name__ + ".kernels.gemm"].REGISTRATIONS
                     if r != eo["registration"]]
        eo["other_registrations"] = [eager_overhead_other_registration(r) for r in other_reg]
        extras["eager_call_overhead"] = eo
        log("eager call host us (" + eo["registration"] + "): " + ", ".join(
            f"{k} {v['host_us']:.2f}" for k, v in eo["rows"].items()))
        for o in eo["other_registrations"]:
            if "rows" in o:
                log(f"  under {o['registration']}: nanovllm::gemm {o['rows']['nanovllm::gemm']['host_us']:.2f} us")

    # ------------------------------------------ vendor comparison (not used)
    if not args.no_vendor:
        F = torch.nn.functional

        def vendor(aa, ww):
            def f():
                F.linear(aa, ww)
            return f
        try:
            if wl.b_layout != L.B_NK:
                raise RuntimeError("vendor comparison is timed for the W[N,K] layout only")
            t_ms = median_graph_ms(torch, [vendor(a, w)] * 200)
            vt = flops / (t_ms * 1e-3) / 1e12
            extras["vendor_torch_linear"] = {"us": round(t_ms * 1e3, 3), "TFLOP/s": round(vt, 2),
                                                     "note": "torch.matmul on the GPU (hipBLASLt/rocBLAS), "
                                                             "comparison only, never dispatched to"}
            log(f"vendor torch F.linear ({name}): {t_ms * 1e3:.2f} us  {vt:.1f} TFLOP/s")
        except Exception as exc:  # comparison only; never fails the bench
            extras["vendor_torch_linear"] = {"error": str(exc)[:200]}

    # ------------------------------------------------------------ CPU baseline
    if not args.no_cpu:
        from oracle import cpu_baseline

        a_cpu, w_cpu = W.make_inputs(name, m)
        cb = cpu_baseline.time_cpu_gemm(a_cpu, w_cpu, wl.b_layout == L.B_NK, wl.dtype_out,
                                        budget_s=args.cpu_budget)
        cpu_tf = flops / cb["seconds"] / 1e12
        call = "F.linear(a, W)" if wl.b_layout == L.B_NK else "torch.matmul(a, B)"
        # kind "reference": the timed call is the reference's own operation
        # (F.linear at nanovllm/layers/linear.py:51, torch.matmul as the FP32
        # ladder's differential target) on PyTorch's CPU kernels, not the
        # oracle's float64 restatement.
        result["cpu_baseline"] = {
            "value": round(cpu_tf, 4), "unit": "TFLOP/s", "cores": cb["threads"], "kind": "reference",
            "sample": f"full {m}x{n}x{k} {dname[wl.dtype_in]} GEMM, torch {call} on the host CPU "
                      f"({cb['cpu_model']}, {cb['threads']} threads of {cb['cpu_count']}), median of "
                      f"{cb['samples']} calls",
        }
        log(f"cpu baseline: {cb['seconds'] * 1e3:.1f} ms/call  {cpu_tf:.3f} TFLOP/s on {cb['threads']} threads")
        # Every configuration of the workload table on the same host, same
        # seeded inputs and dtypes (TFLOP/s and GB/s of the same algorithmic
        # work as the GPU rows).
        rows_cpu = []
        for cname, cw in W.WORKLOADS.items():
            for cm in cw.ms:
                a_c, b_c = W.make_inputs(cname, cm)
                cbc = cpu_baseline.time_cpu_gemm(a_c, b_c, cw.b_layout == L.B_NK, cw.dtype_out,
                                                 budget_s=max(1.0, args.cpu_budget / 4))
                fl = W.problem_flops(cm, cw.n, cw.k)
                by = W.problem_bytes(cm, cw.n, cw.k, cw.dtype_in, cw.dtype_out)
                rows_cpu.append({"workload": cname, "m": cm, "ms_per_call": round(cbc["seconds"] * 1e3, 4),
                                 "TFLOP/s": round(fl / cbc["seconds"] / 1e12, 4),
                                 "GB/s": round(by / cbc["seconds"] / 1e9, 2), "samples": cbc["samples"],
                                 "call": "F.linear" if cw.b_layout == L.B_NK else "torch.matmul"})
                log(f"cpu baseline {cname} M={cm}: {cbc['seconds'] * 1e3:.2f} ms/call")
                del a_c, b_c
        extras["cpu_baseline_configs"] = {"kind": "reference", "cores": cb["threads"], "cpu_model": cb["cpu_model"],
                                          "cpu_count": cb["cpu_count"], "rows": rows_cpu}

    result.update(extras)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
