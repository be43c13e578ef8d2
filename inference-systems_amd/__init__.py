"""MI355X-native shape-aware GEMM for nano-vLLM linear layers.

Importable as ``inference_systems_amd`` (the directory name carries a
hyphen, so it is registered under that name by the loaders in
``__graft_entry__.py`` and ``tests/conftest.py``).

  _lib      ctypes binding of libnanovllm_gemm.so (the C ABI)
  kernels   the ``nanovllm::gemm`` / ``nanovllm::gemm_kn`` torch ops
  layers    nano-vLLM Linear / LM-head classes routed through the op
  workloads the measured GEMM shapes and their synthetic inputs
  build     hipcc recipe for the library
"""
from . import _lib, layers, workloads
from .kernels import gemm, gemm_kn, gemm_with_kernel, linear, selected_kernel

__all__ = ["_lib", "layers", "workloads", "gemm", "gemm_kn", "gemm_with_kernel", "linear", "selected_kernel"]
