"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

capi.cpp (argument validation, the selection table, workspace sizes, the
thread-local error message) is rebuilt with host-only ASan + UBSan into a
temporary directory, and the CPU tests of the C ABI (tests/test_capi.py) run
against that copy in a child process with the sanitizer runtime preloaded.
The reference ran its kernels under compute-sanitizer memcheck / racecheck
(cuda_kernels/gemm/README.md:157-169); the host-side counterpart here is
the part a sanitizer can cover without a GPU-instrumented build.  No kernel is launched.
"""
from __future__ import annotations

import importlib.util
import os
import subprocess
import sys

import pytest

from conftest import ROOT

CHILD = r"""
import sys
maps = open("/proc/self/maps").read()
assert "libclang_rt.asan" in maps, "sanitizer runtime not preloaded"
import pytest
sys.path.insert(0, {root!r})
rc = pytest.main(["-q", "-m", "not gpu", "-p", "no:cacheprovider", {tests!r}])
sys.path.insert(0, {root!r} + "/tests")
from conftest import PKG
import os
loaded = PKG._lib.library_path()
assert str(loaded) == os.environ["NANOVLLM_GEMM_LIB"], loaded
assert str(loaded) in open("/proc/self/maps").read(), "sanitized library not mapped"
sys.exit(int(rc))
"""


def _build_module():
    spec = importlib.util.spec_from_file_location("_nvgemm_build_san", ROOT / "inference-systems_amd" / "build.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_capi_under_asan_ubsan(tmp_path):
    build = _build_module()
    try:
        runtime = build.sanitizer_runtime()
        build.hipcc()
    except RuntimeError as exc:
        pytest.skip(str(exc))
    lib = build.build(sanitize=True, out=tmp_path / "libnanovllm_gemm.so")
    undefined = subprocess.run(["nm", "-D", "--undefined-only", str(lib)], capture_output=True, text=True).stdout
    assert "__asan_report" in undefined and "__ubsan_handle" in undefined, "capi.cpp was not instrumented"
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": str(runtime),
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "NANOVLLM_GEMM_LIB": str(lib),
    })
    code = CHILD.format(root=str(ROOT), tests=str(ROOT / "tests" / "test_capi.py"))
    proc = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=600,
                          cwd=str(tmp_path))
    out = proc.stdout + proc.stderr
    assert proc.returncode == 0, out[-4000:]
    assert "passed" in proc.stdout and "failed" not in proc.stdout, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
