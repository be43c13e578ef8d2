"""Build recipe for libnanovllm_gemm.so (hipcc, gfx950 only).

Every HIP source under csrc/ is compiled to an object in a temporary
directory, in parallel, and linked into ``libnanovllm_gemm.so`` next to this
file.  The library is loaded with ctypes by ``_lib.py``; it has no
dependency on torch.

Usage: ``python inference-systems_amd/build.py`` or ``build()`` from Python.
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
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
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


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every source and link the shared library; returns its path."""
    extra = list(extra_flags or [])
    with tempfile.TemporaryDirectory(prefix="nvgemm_build_") as tmp:
        tmpdir = Path(tmp)
        jobs = []
        with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4, 8)) as pool:
            for name in SOURCES:
                src = CSRC / name
                obj = tmpdir / (name + ".o")
                jobs.append((obj, pool.submit(_compile, src, obj, extra)))
            for _, fut in jobs:
                fut.result()
        out_tmp = tmpdir / LIB_NAME
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(out_tmp),
               *[str(o) for o, _ in jobs]]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stderr}")
        # Replace atomically so a process that has the old file mapped keeps it.
        final_tmp = LIB_PATH.with_suffix(".so.tmp")
        shutil.copyfile(out_tmp, final_tmp)
        os.replace(final_tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
