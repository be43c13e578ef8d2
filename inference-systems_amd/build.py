"""Build recipe for libnanovllm_gemm.so (hipcc, gfx950 only).

Every HIP source under csrc/ is compiled to an object in a temporary
directory, in parallel, and linked into ``libnanovllm_gemm.so`` next to this
file.  The library is loaded with ctypes by ``_lib.py``; it has no
dependency on torch.  ``libnanovllm_torch_ops.so`` (csrc/torch_ops.cpp, host
C++ against PyTorch's headers) registers nanovllm::gemm / gemm_kn from C++
over that library.

Usage: ``python inference-systems_amd/build.py`` or ``build()`` from Python;
``build.py --resource-usage [KERNEL_STATS_CSV]`` prints every kernel's
registers, LDS, spills and occupancy from the compiler's
kernel-resource-usage remarks (with a rocprofv3 kernel-stats CSV: per family,
and for each kernel that run launched).

``build(sanitize=True, out=path)`` (``build.py --sanitize PATH``) builds a
copy whose host code in capi.cpp (argument validation, the selection table,
workspace sizes, error reporting) carries AddressSanitizer and
UndefinedBehaviorSanitizer; device code is built as usual.  It is loaded
through ``NANOVLLM_GEMM_LIB`` with the sanitizer runtime preloaded
(``sanitizer_runtime()``), for the CPU tests of the C ABI.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libnanovllm_gemm.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
# -amdgpu-kernarg-preload-count=16: the first 16 SGPRs of kernel arguments
# arrive preloaded, so a kernel's first copies wait for no argument load
# (the kernels put the arguments those copies need first).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]

SOURCES = [
    "capi.cpp",
    "gemm_fp32.hip",
    "gemm_direct.hip",
    "gemm_staged.hip",
    "gemm_decode.hip",
    "gemm_gemv.hip",
    "gemm_argmax.hip",
    "gemm_prologue.hip",
]

# The microbenchmarks behind `bench.py --probes` and the decode
# configuration sweep behind `bench.py --decode-sweep`: libraries of their
# own, so the GEMM library carries only the product's entry points.
PROBE_SOURCES = ["probes.hip"]
PROBE_LIB_PATH = PKG_DIR / "libnanovllm_probes.so"
SWEEP_SOURCES = ["decode_sweep.hip"]
SWEEP_LIB_PATH = PKG_DIR / "libnanovllm_decode_sweep.so"

# The C++ registration of nanovllm::gemm / gemm_kn (TORCH_LIBRARY over the
# C ABI): host code only, built with the host compiler against PyTorch's
# headers and linked to libnanovllm_gemm.so next to it.
TORCH_OPS_SOURCE = "torch_ops.cpp"
TORCH_OPS_LIB_PATH = PKG_DIR / "libnanovllm_torch_ops.so"
INCLUDE_DIR = PKG_DIR.parent / "include"


# Host-only sanitizers for capi.cpp: each -fsanitize= goes to the host pass
# alone (-Xarch_host), so no GPU code is instrumented.
SANITIZE_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-g",
]
SANITIZED_SOURCES = ("capi.cpp",)


def sanitizer_runtime() -> Path:
    """The ASan runtime of the ROCm clang that built the sanitized library
    (it carries the UBSan handlers too); preloaded into the Python that loads it."""
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    found = sorted((rocm / "llvm" / "lib" / "clang").glob("*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not found:
        raise RuntimeError("libclang_rt.asan-x86_64.so not found under the ROCm clang")
    return found[-1]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: the gfx950 GEMM library needs the ROCm toolchain")
    return found


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), "-x", "hip", *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know -packed-fp32-ops; drop
    # only that line.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, extra_flags: list[str] | None = None, sanitize: bool = False,
          out: Path | None = None) -> Path:
    """Compile every source and link the shared library; returns its path.

    sanitize: capi.cpp's host code with ASan + UBSan (needs `out`, so the
    in-tree library is never replaced by an instrumented one)."""
    extra = list(extra_flags or [])
    if sanitize and out is None:
        raise ValueError("a sanitized build needs an output path outside the package")
    target = Path(out) if out is not None else LIB_PATH
    with tempfile.TemporaryDirectory(prefix="nvgemm_build_") as tmp:
        tmpdir = Path(tmp)
        jobs = []
        with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4, 8)) as pool:
            for name in SOURCES:
                src = CSRC / name
                obj = tmpdir / (name + ".o")
                flags = extra + (SANITIZE_FLAGS if sanitize and name in SANITIZED_SOURCES else [])
                jobs.append((obj, pool.submit(_compile, src, obj, flags)))
            for _, fut in jobs:
                fut.result()
        out_tmp = tmpdir / LIB_NAME
        # A sanitized library leaves the runtime's symbols undefined: the
        # runtime is preloaded into the process that loads it.
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(out_tmp),
               *[str(o) for o, _ in jobs]]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stderr}")
        # Replace atomically so a process that has the old file mapped keeps it.
        target.parent.mkdir(parents=True, exist_ok=True)
        final_tmp = target.with_suffix(".so.tmp")
        shutil.copyfile(out_tmp, final_tmp)
        os.replace(final_tmp, target)
    if verbose:
        print(f"built {target}")
    if not sanitize and out is None:
        build_probes(verbose=verbose, extra_flags=extra)
        build_torch_ops(verbose=verbose)
    return target


def build_torch_ops(verbose: bool = False) -> Path:
    """Compile csrc/torch_ops.cpp into libnanovllm_torch_ops.so (needs the
    in-tree libnanovllm_gemm.so, found at run time through $ORIGIN)."""
    import torch

    if not LIB_PATH.is_file():
        raise RuntimeError(f"{LIB_NAME} must be built before {TORCH_OPS_LIB_PATH.name}")
    tdir = Path(torch.__file__).resolve().parent
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    with tempfile.TemporaryDirectory(prefix="nvgemm_tops_") as tmp:
        out_tmp = Path(tmp) / TORCH_OPS_LIB_PATH.name
        cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
               "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
               f"-I{tdir / 'include'}", f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
               f"-I{rocm}/include", f"-I{INCLUDE_DIR}",
               str(CSRC / TORCH_OPS_SOURCE), "-o", str(out_tmp),
               f"-L{PKG_DIR}", "-lnanovllm_gemm", f"-L{tdir / 'lib'}", "-lc10", "-lc10_hip", "-ltorch",
               "-ltorch_cpu", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tdir / 'lib'}"]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"building {TORCH_OPS_LIB_PATH.name} failed:\n{proc.stderr}")
        final_tmp = TORCH_OPS_LIB_PATH.with_suffix(".so.tmp")
        shutil.copyfile(out_tmp, final_tmp)
        os.replace(final_tmp, TORCH_OPS_LIB_PATH)
    if verbose:
        print(f"built {TORCH_OPS_LIB_PATH}")
    return TORCH_OPS_LIB_PATH


def _build_aux(sources: list[str], lib_path: Path, verbose: bool, extra_flags: list[str] | None) -> Path:
    with tempfile.TemporaryDirectory(prefix="nvgemm_aux_") as tmp:
        out_tmp = Path(tmp) / lib_path.name
        cmd = [hipcc(), "-x", "hip", *HIP_FLAGS, *(extra_flags or []), "-shared", "-o", str(out_tmp),
               *[str(CSRC / name) for name in sources]]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        noise = "'-packed-fp32-ops' is not a recognized feature"
        err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {lib_path.name}:\n{err}")
        final_tmp = lib_path.with_suffix(".so.tmp")
        shutil.copyfile(out_tmp, final_tmp)
        os.replace(final_tmp, lib_path)
    if verbose:
        print(f"built {lib_path}")
    return lib_path


def build_probes(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile the microbenchmark library (libnanovllm_probes.so) and the
    decode configuration sweep (libnanovllm_decode_sweep.so)."""
    with ThreadPoolExecutor(max_workers=2) as pool:
        jobs = [pool.submit(_build_aux, PROBE_SOURCES, PROBE_LIB_PATH, verbose, extra_flags),
                pool.submit(_build_aux, SWEEP_SOURCES, SWEEP_LIB_PATH, verbose, extra_flags)]
        for j in jobs:
            j.result()
    return PROBE_LIB_PATH


_REMARK_KEYS = {"VGPRs": "vgpr", "AGPRs": "agpr", "TotalSGPRs": "sgpr", "ScratchSize [bytes/lane]": "scratch",
                "Occupancy [waves/SIMD]": "occupancy", "SGPRs Spill": "sgpr_spill", "VGPRs Spill": "vgpr_spill",
                "LDS Size [bytes/block]": "lds"}


def resource_usage(sources: list[str] | None = None) -> list[dict]:
    """Per kernel of the GEMM library: VGPRs, AGPRs, SGPRs, scratch, spills,
    static LDS and the compiler's occupancy (waves per SIMD), from the gfx950
    device pass's kernel-resource-usage remarks; kernel names demangled."""
    import re

    rows = []
    for name in sources or [n for n in SOURCES if n.endswith(".hip")]:
        cmd = [hipcc(), "-x", "hip", *HIP_FLAGS, "--offload-device-only", "-Rpass-analysis=kernel-resource-usage",
               "-c", str(CSRC / name), "-o", os.devnull]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed for {name}:\n{proc.stderr[-2000:]}")
        cur = None
        for line in proc.stderr.splitlines():
            m = re.search(r"remark: Function Name: (\S+)", line)
            if m:
                cur = {"source": name, "mangled": m.group(1)}
                rows.append(cur)
                continue
            m = re.search(r"remark:\s+([^:]+): (\S+) \[-Rpass-analysis", line)
            if m and cur is not None and m.group(1).strip() in _REMARK_KEYS:
                val = m.group(2)
                cur[_REMARK_KEYS[m.group(1).strip()]] = int(val) if val.lstrip("-").isdigit() else val
    if rows:
        demangled = subprocess.run(["c++filt"], input="\n".join(r["mangled"] for r in rows), capture_output=True,
                                   text=True).stdout.splitlines()
        for r, d in zip(rows, demangled):
            r["kernel"] = re.sub(r"^(void )?nvg::\(anonymous namespace\)::", "", d).replace("(anonymous namespace)::", "")
    return rows


def resource_table(rows: list[dict]) -> str:
    lines = ["| source | kernel | VGPR | AGPR | SGPR | LDS bytes | occupancy (waves/SIMD) | VGPR / SGPR spills | "
             "scratch bytes/lane |", "|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        kern = r["kernel"].split("(")[0] if "(" in r["kernel"] else r["kernel"]
        lines.append(f"| {r['source']} | `{kern}` | {r.get('vgpr')} | {r.get('agpr')} | {r.get('sgpr')} | "
                     f"{r.get('lds')} | {r.get('occupancy')} | {r.get('vgpr_spill')} / {r.get('sgpr_spill')} | "
                     f"{r.get('scratch')} |")
    return "\n".join(lines)


def _short_name(name: str) -> str:
    """`mfma_staged_kernel<2, 2, 128, 256, ...>` from a demangled name with
    namespace, return type and parameter list."""
    import re

    name = re.sub(r"^void ", "", name).replace("nvg::", "").replace("(anonymous namespace)::", "")
    depth = 0
    for i, ch in enumerate(name):
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            return name[:i]
    return name


def resource_report(rows: list[dict], stats_csv: Path | None = None) -> str:
    """Markdown: per kernel family the number of instantiations and the range
    of each resource; with a rocprofv3 kernel-stats CSV, one row per library
    kernel that run launched (calls, average duration, resources)."""
    import csv
    from collections import defaultdict

    fam = defaultdict(list)
    for r in rows:
        fam[_short_name(r["kernel"]).split("<")[0]].append(r)

    def rng(v, key):
        lo, hi = min(x.get(key, 0) for x in v), max(x.get(key, 0) for x in v)
        return f"{lo}" if lo == hi else f"{lo}-{hi}"
    out = ["| family | instantiations | VGPR | AGPR | LDS bytes | occupancy (waves/SIMD) | spills (VGPR / SGPR) | "
           "scratch |", "|---|---|---|---|---|---|---|---|"]
    for f, v in fam.items():
        out.append(f"| `{f}` | {len(v)} | {rng(v, 'vgpr')} | {rng(v, 'agpr')} | {rng(v, 'lds')} | "
                   f"{rng(v, 'occupancy')} | {rng(v, 'vgpr_spill')} / {rng(v, 'sgpr_spill')} | {rng(v, 'scratch')} |")
    if stats_csv is not None:
        by_name = {_short_name(r["kernel"]): r for r in rows}
        traced = []
        with open(stats_csv, newline="") as fh:
            for st in csv.DictReader(fh):
                key = _short_name(st["Name"])
                if key in by_name:
                    traced.append((key, int(st["Calls"]), float(st["AverageNs"]) / 1e3, by_name[key]))
        traced.sort(key=lambda t: (t[0].split("<")[0], -t[1]))
        out += ["", "| kernel (as launched) | calls | average us | VGPR | AGPR | SGPR | LDS bytes | "
                    "workgroups per CU by LDS | occupancy (waves/SIMD) | spills |",
                "|---|---|---|---|---|---|---|---|---|---|"]
        for key, calls, avg, r in traced:
            wg_lds = 163840 // r["lds"] if r.get("lds") else "-"
            out.append(f"| `{key}` | {calls} | {avg:.2f} | {r.get('vgpr')} | {r.get('agpr')} | {r.get('sgpr')} | "
                       f"{r.get('lds')} | {wg_lds} | {r.get('occupancy')} | "
                       f"{r.get('vgpr_spill')} / {r.get('sgpr_spill')} |")
    return "\n".join(out)


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--sanitize":
        build(verbose=True, sanitize=True, out=Path(sys.argv[2]))
    elif len(sys.argv) in (2, 3) and sys.argv[1] == "--resource-usage":
        # --resource-usage [KERNEL_STATS_CSV]: every kernel's resources; with
        # a rocprofv3 kernel-stats CSV, the summary per family and one row
        # per kernel that run launched.
        usage = resource_usage()
        if len(sys.argv) == 3:
            print(resource_report(usage, Path(sys.argv[2])))
        else:
            print(resource_table(usage))
    else:
        build(verbose=True)
