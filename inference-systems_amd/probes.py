"""Microbenchmarks of the MI355X ceilings the GEMM kernels are measured
against (csrc/probes.hip, built into libnanovllm_probes.so), run by
``bench.py --probes``.

Each probe returns one figure of the hardware on the box it runs on: the
launch floor of a kernel node in a HIP graph, the streaming read rate of
HBM, the LDS read rate, the global -> LDS copy rate of the copy instruction
the GEMM kernels use (and of the register-staged alternatives), the bf16
MFMA rate, and the shader clock under each load (from the s_memtime and
s_memrealtime stamps of one wave).
"""
from __future__ import annotations

import ctypes
import math
import statistics
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libnanovllm_probes.so"
REALTIME_HZ = 100e6          # s_memrealtime counts at 100 MHz
CUS = 256

_I64, _INT, _VP = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p
_SIGS = {
    "nvprobe_empty": [_INT, _VP],
    "nvprobe_stream_read": [_VP, _I64, _INT, _INT, _VP, _VP, _VP],
    "nvprobe_lds_read": [_INT, _INT, _VP, _VP, _VP],
    "nvprobe_copy": [_INT, _VP, _I64, _INT, _INT, _INT, _INT, _VP, _VP, _VP],
    "nvprobe_mfma": [_INT, _INT, _INT, _VP, _VP, _VP],
    "nvprobe_mfma16": [_INT, _INT, _INT, _VP, _VP, _VP],
    "nvprobe_write_tiles": [_VP, _I64, _INT, _INT, _INT, _VP, _VP],
    "nvprobe_lds_map": [_VP, _INT, _INT, _INT, _INT, _VP, _VP, _VP],
}
_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise RuntimeError(f"{LIB_PATH.name} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, args in _SIGS.items():
            getattr(lib, name).restype = _INT
            getattr(lib, name).argtypes = args
        _lib = lib
    return _lib


def _check(rc, what):
    if rc != 0:
        raise RuntimeError(f"probe {what} refused its arguments or failed to launch")


class _Ctx:
    """Sink and clock buffers on the device, and event timing on the current stream."""

    def __init__(self, torch, max_workgroups):
        self.torch = torch
        self.sink = torch.zeros(8 * max_workgroups, dtype=torch.int32, device="cuda")
        self.clocks = torch.zeros(4, dtype=torch.int64, device="cuda")

    def stream(self):
        return self.torch.cuda.current_stream().cuda_stream

    def time_ms(self, launch, reps=5):
        t = self.torch
        launch()
        t.cuda.synchronize()
        samples = []
        for _ in range(reps):
            s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
            s.record()
            launch()
            e.record()
            t.cuda.synchronize()
            samples.append(s.elapsed_time(e))
        return statistics.median(samples)

    def clock_ghz(self):
        """Shader clock of the last launch, from wave 0 of workgroup 0."""
        c = self.clocks.cpu().tolist()
        d_t, d_r = c[2] - c[0], c[3] - c[1]
        return (d_t / d_r) * REALTIME_HZ / 1e9 if d_r > 0 else math.nan


def launch_floor(torch, launches=1000):
    """Per-node time of a HIP graph of empty kernels, and per launch from the stream."""
    lib = load()
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    _check(lib.nvprobe_empty(1, stream()), "empty")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _check(lib.nvprobe_empty(launches, stream()), "empty")
    ctx = _Ctx(torch, 1)
    graph_ms = ctx.time_ms(g.replay)
    plain_ms = ctx.time_ms(lambda: _check(lib.nvprobe_empty(launches, stream()), "empty"))
    return {"graph_node_us": 1e3 * graph_ms / launches, "stream_launch_us": 1e3 * plain_ms / launches,
            "launches": launches}


def stream_read(torch, nbytes, copies, per_lane_list=(1, 2, 4, 8), reps_per_copy=4):
    """Graph replays of a streaming read of an `nbytes` buffer rotated over
    `copies` copies (each launch reads one copy, so reads come from HBM once
    the copies exceed the Infinity Cache)."""
    lib = load()
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i) for i in range(copies)]
    rows = []
    for pl in per_lane_list:
        wgs = nbytes // (256 * 16 * pl)
        if wgs * 256 * 16 * pl != nbytes:
            continue
        ctx = _Ctx(torch, wgs)
        launches = []
        for i in range(copies * reps_per_copy):
            b = bufs[i % copies]
            launches.append((b.data_ptr(), wgs, pl))

        def run():
            s = ctx.stream()
            for ptr, w, p in launches:
                _check(lib.nvprobe_stream_read(ptr, nbytes, w, p, ctx.sink.data_ptr(), None, s), "stream_read")
        run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run()
        for _ in range(3):
            g.replay()
        us = 1e3 * ctx.time_ms(g.replay) / len(launches)
        rows.append({"bytes": nbytes, "workgroups": wgs, "loads_per_lane": pl, "us": round(us, 3),
                     "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1)})
    del bufs
    return rows


def lds_read(torch, workgroups=CUS, iters=1024):
    lib = load()
    ctx = _Ctx(torch, workgroups)
    run = lambda: _check(lib.nvprobe_lds_read(workgroups, iters, ctx.sink.data_ptr(), ctx.clocks.data_ptr(),  # noqa
                                              ctx.stream()), "lds_read")
    ms = ctx.time_ms(run)
    ghz = ctx.clock_ghz()
    nbytes = workgroups * 8 * iters * 1024
    per_cu = nbytes / min(workgroups, CUS) if workgroups <= CUS else nbytes / CUS
    return {"workgroups": workgroups, "bytes": nbytes, "us": round(ms * 1e3, 2), "clock_ghz": round(ghz, 3),
            "bytes_per_clk_per_cu": round(per_cu / (ms * 1e-3 * ghz * 1e9), 1)}


COPY_MODES = {0: "global_load_lds_dwordx4 (to LDS)", 1: "global_load_dwordx4 (to VGPRs)",
              2: "global_load_dwordx4 + ds_write_b128 (to LDS through VGPRs)",
              3: "half the waves each of modes 0 and 2 (to LDS)"}


def copy_rate(torch, mode, workgroups=CUS, iters=512, inflight=8, window=4 << 20, reads=0):
    """Copy rate of one copy path; with reads = 3, three 1 KiB ds_read_b128
    per copied KiB share the LDS (bytes_per_clk_per_cu counts the copies)."""
    lib = load()
    ctx = _Ctx(torch, workgroups)
    src = torch.ones(window, dtype=torch.uint8, device="cuda")
    run = lambda: _check(lib.nvprobe_copy(mode, src.data_ptr(), window, workgroups, iters, inflight, reads,  # noqa
                                          ctx.sink.data_ptr(), ctx.clocks.data_ptr(), ctx.stream()), "copy")
    ms = ctx.time_ms(run)
    ghz = ctx.clock_ghz()
    nbytes = workgroups * 8 * iters * 1024
    return {"mode": COPY_MODES[mode], "workgroups": workgroups, "inflight_per_wave": inflight,
            "lds_reads_per_copy": reads, "window_bytes": window, "bytes": nbytes, "us": round(ms * 1e3, 2),
            "clock_ghz": round(ghz, 3), "bytes_per_clk_per_cu": round(nbytes / CUS / (ms * 1e-3 * ghz * 1e9), 1),
            "TB/s": round(nbytes / (ms * 1e-3) / 1e12, 2)}


def mfma_rate(torch, workgroups=CUS, iters=2048, chains=4, shape="32x32x16"):
    """bf16 MFMA throughput: 8 waves per workgroup, `chains` independent
    accumulators per wave, v_mfma_f32_32x32x16_bf16 or (shape "16x16x32")
    v_mfma_f32_16x16x32_bf16, whose instruction has a quarter of the flops."""
    lib = load()
    ctx = _Ctx(torch, workgroups)
    entry = lib.nvprobe_mfma if shape == "32x32x16" else lib.nvprobe_mfma16
    if shape == "16x16x32":
        iters *= 4   # the same flops per wave
    run = lambda: _check(entry(workgroups, iters, chains, ctx.sink.data_ptr(), ctx.clocks.data_ptr(),  # noqa
                               ctx.stream()), "mfma")
    ms = ctx.time_ms(run)
    ghz = ctx.clock_ghz()
    per_instr = 32 * 32 * 16 if shape == "32x32x16" else 16 * 16 * 32
    flops = workgroups * 8 * iters * chains * 2.0 * per_instr
    return {"shape": shape, "workgroups": workgroups, "chains": chains, "us": round(ms * 1e3, 2),
            "clock_ghz": round(ghz, 3),
            "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
            "peak_at_clock_TFLOP/s": round(2500.0 * ghz / 2.4, 1)}


def write_tiles(torch, rows=2048, cols_bytes=8192, nontemporal=True, copies=1, reps=200):
    """Graph replays of a kernel that writes every 128 x 512-byte tile of a
    rows x cols_bytes matrix (the C tiles of the 2048 x 4096 bf16 GEMM), one
    512-thread workgroup per tile; `copies` output buffers in rotation."""
    lib = load()
    tiles_m, tiles_n = rows // 128, cols_bytes // 512
    nbytes = rows * cols_bytes
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    ctx = _Ctx(torch, 1)

    def run():
        s = ctx.stream()
        for i in range(reps):
            _check(lib.nvprobe_write_tiles(bufs[i % copies].data_ptr(), cols_bytes, tiles_m, tiles_n,
                                           int(nontemporal), None, s), "write_tiles")
    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    g.replay()
    us = 1e3 * ctx.time_ms(g.replay) / reps
    return {"bytes": nbytes, "workgroups": tiles_m * tiles_n, "nontemporal": nontemporal, "buffers": copies,
            "us": round(us, 3), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1)}


# ---------------------------------------------------------------------------
# Decode configuration sweep (csrc/decode_sweep.hip, libnanovllm_decode_sweep.so)
# ---------------------------------------------------------------------------
SWEEP_LIB_PATH = Path(__file__).resolve().parent / "libnanovllm_decode_sweep.so"
_sweep = None


def load_sweep():
    global _sweep
    if _sweep is None:
        if not SWEEP_LIB_PATH.is_file():
            raise RuntimeError(f"{SWEEP_LIB_PATH.name} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(str(SWEEP_LIB_PATH))
        lib.nvsweep_decode_count.restype = _INT
        lib.nvsweep_decode_count.argtypes = []
        lib.nvsweep_decode_name.restype = ctypes.c_char_p
        lib.nvsweep_decode_name.argtypes = [_INT]
        lib.nvsweep_decode_max_m.restype = _INT
        lib.nvsweep_decode_max_m.argtypes = [_INT]
        lib.nvsweep_decode_kn.restype = _INT
        lib.nvsweep_decode_kn.argtypes = [_INT]
        lib.nvsweep_decode.restype = _INT
        lib.nvsweep_decode.argtypes = [_INT, _VP, _VP, _VP, _I64, _I64, _I64, _VP]
        _sweep = lib
    return _sweep


def sweep_configs():
    """(index, name, max M, B[K,N]?) of every decode configuration in the sweep library."""
    lib = load_sweep()
    return [(i, lib.nvsweep_decode_name(i).decode(), lib.nvsweep_decode_max_m(i), lib.nvsweep_decode_kn(i) == 1)
            for i in range(lib.nvsweep_decode_count())]


def sweep_launcher(torch, cfg, a, w, c):
    """A no-argument launch of configuration `cfg` on bf16 a[M,K] and w (W[N,K],
    or B[K,N] for a B[K,N] configuration) into c[M,N]."""
    lib = load_sweep()
    m, k = a.shape
    n = c.shape[1]
    args = (cfg, a.data_ptr(), w.data_ptr(), c.data_ptr(), m, n, k)

    def f():
        _check(lib.nvsweep_decode(*args, torch.cuda.current_stream().cuda_stream), "decode sweep")
    return f


def lds_map_cycles(torch, offsets, width, write=False, workgroups=CUS, iters=4096):
    """LDS clocks per instruction of a CU when its four waves each issue
    `iters` instructions of `width` bytes per lane, lane L at byte offset
    offsets[L] (median over the workgroups, one per CU)."""
    lib = load()
    if len(offsets) != 64:
        raise ValueError("one offset per lane")
    arr = (ctypes.c_uint32 * 64)(*offsets)
    sink = torch.zeros(8 * workgroups, dtype=torch.int32, device="cuda")
    cycles = torch.zeros(workgroups, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(2):   # the first launch warms the clocks
        _check(lib.nvprobe_lds_map(arr, width, int(write), workgroups, iters, sink.data_ptr(), cycles.data_ptr(),
                                   stream), "lds_map")
    torch.cuda.synchronize()
    return statistics.median(cycles.cpu().tolist()) / (4 * iters)


def _pack(lane, bits):
    return sum(((lane >> b) & 1) << i for i, b in enumerate(bits))


def lds_lane_groups(torch):
    """Which lanes the LDS serves together.  Lane L owns 256-byte row L (so
    every lane reads its own address) and picks its column from the lane
    bits in `bits`: the maps whose chosen bits are exactly the bits that vary
    inside the group the LDS serves per clock take the fewest clocks.  Also
    all lanes on one column (the worst case) and, for 16-byte accesses, the
    fragment-read map of the fp32 kernel (16 rows, lane group l / 16 at
    chunk 4 (l / 16) ^ row)."""
    from itertools import combinations

    out = {}
    for width, nbits in ((16, 4), (8, 5), (4, 6)):
        rows = {}
        for write in (False, True):
            res = {}
            for bits in combinations(range(6), nbits):
                offs = [lane * 256 + _pack(lane, bits) * width for lane in range(64)]
                res["bits " + "".join(str(b) for b in bits)] = lds_map_cycles(torch, offs, width, write)
            res["one column"] = lds_map_cycles(torch, [lane * 256 for lane in range(64)], width, write)
            if width == 16:
                offs = [(lane % 16) * 256 + ((4 * (lane // 16)) ^ (lane % 16)) * 16 for lane in range(64)]
                res["fp32 fragment map"] = lds_map_cycles(torch, offs, width, write)
            rows["write" if write else "read"] = {k: round(v, 3) for k, v in res.items()}
        out[f"b{8 * width}"] = rows
    return out
