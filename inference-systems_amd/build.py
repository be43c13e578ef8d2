"""Build recipe for libnanovllm_gemm.so (hipcc, gfx950 only).

Every HIP source under csrc/ is compiled to an object in a temporary
directory, in parallel, and linked into ``libnanovllm_gemm.so`` next to this
file.  The library is loaded with ctypes by ``_lib.py``; it has no
dependency on torch.  ``libnanovllm_torch_ops.so`` (csrc/torch_ops.cpp, host
C++ against PyTorch's headers) registers nanovllm::gemm / gemm_kn from C++
over that library.

Usage: ``python inference-systems_amd/build.py`` or ``build()`` from Python.

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


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--sanitize":
        build(verbose=True, sanitize=True, out=Path(sys.argv[2]))
    else:
        build(verbose=True)
