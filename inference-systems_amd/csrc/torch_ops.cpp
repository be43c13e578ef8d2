// torch_ops.cpp — nanovllm::gemm and nanovllm::gemm_kn registered from C++.
//
// The registration pattern of nanovllm/csrc/ops.cpp:48-80 (TORCH_LIBRARY
// block, one CUDA-key implementation per op) over the C ABI of
// libnanovllm_gemm.so: the op checks its arguments, allocates the output
// with the input's options and enqueues the GEMM on PyTorch's current HIP
// stream of the input's device, so it is graph-capturable like the
// reference's add op (nanovllm/csrc/add_kernel.cu:49-67).
//
// The argument contract and its messages are those of the Python
// registration (kernels/gemm.py: contract_reason), so callers see the same
// RuntimeError text from either registration; the schemas are identical.
// The fake (meta) implementations stay in Python (torch.library.register_fake).
//
// What this file buys over the ctypes + torch.library.custom_op
// registration is the host cost of one eager call: the dispatcher reaches
// C++ directly instead of going through the Python custom-op machinery,
// ctypes argument conversion and Python-side checks.

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <optional>
#include <string>

#include "nanovllm_gemm.h"

namespace {

int dtype_code(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return NANOVLLM_GEMM_F32;
        case at::kHalf: return NANOVLLM_GEMM_F16;
        case at::kBFloat16: return NANOVLLM_GEMM_BF16;
        default: return -1;
    }
}

// torch's Python spelling of a dtype ("torch.bfloat16"), for messages.
std::string dtype_name(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return "torch.float32";
        case at::kHalf: return "torch.float16";
        case at::kBFloat16: return "torch.bfloat16";
        case at::kDouble: return "torch.float64";
        case at::kLong: return "torch.int64";
        case at::kInt: return "torch.int32";
        case at::kShort: return "torch.int16";
        case at::kChar: return "torch.int8";
        case at::kByte: return "torch.uint8";
        case at::kBool: return "torch.bool";
        default: return std::string("torch.") + c10::toString(t);
    }
}

bool out_ok(at::ScalarType in, at::ScalarType out) {
    if (in == at::kFloat) return out == at::kFloat;
    return out == in || out == at::kFloat;
}

// Why the op cannot take these operands ("" if it can), in the order and
// wording of the Python contract.
std::string contract_reason(const at::Tensor& a, const at::Tensor& b, std::optional<at::ScalarType> out_dtype,
                            int layout) {
    if (!(a.is_cuda() && b.is_cuda())) return "a and w must be CUDA (HIP) tensors";
    if (a.device() != b.device()) return "a and w must be on the same device";
    if (dtype_code(a.scalar_type()) < 0) return "a must be float32, float16 or bfloat16";
    if (b.scalar_type() != a.scalar_type()) return "a and w must have the same dtype";
    const at::ScalarType od = out_dtype.value_or(a.scalar_type());
    if (!out_ok(a.scalar_type(), od)) {
        return "out_dtype " + dtype_name(od) + " is not supported for " + dtype_name(a.scalar_type()) + " inputs";
    }
    if (b.dim() != 2) return "w must be 2-D";
    if (a.dim() < 1) return "a must have at least one dimension";
    const int64_t k = layout == NANOVLLM_GEMM_B_NK ? b.size(1) : b.size(0);
    if (a.size(-1) != k) {
        return "a.size(-1) (" + std::to_string(a.size(-1)) + ") must equal " +
               (layout == NANOVLLM_GEMM_B_NK ? "w.size(1)" : "b.size(0)") + " (" + std::to_string(k) + ")";
    }
    if (k == 0) return "K must be positive";
    if (!a.is_contiguous()) return "a must be contiguous";
    if (!b.is_contiguous()) return "w must be contiguous";
    return {};
}

at::Tensor launch(const at::Tensor& a, const at::Tensor& b, std::optional<at::ScalarType> out_dtype, int layout) {
    const std::string reason = contract_reason(a, b, out_dtype, layout);
    TORCH_CHECK(reason.empty(), "nanovllm::gemm: ", reason);
    const at::ScalarType od = out_dtype.value_or(a.scalar_type());
    const int64_t k = a.size(-1);
    const int64_t n = layout == NANOVLLM_GEMM_B_NK ? b.size(0) : b.size(1);
    const int64_t m = a.numel() / k;
    std::vector<int64_t> sizes = a.sizes().vec();
    sizes.back() = n;
    at::Tensor out = at::empty(sizes, a.options().dtype(od));
    if (m == 0 || n == 0) return out;
    const c10::DeviceGuard guard(a.device());
    hipStream_t stream = c10::hip::getCurrentHIPStream(a.device().index()).stream();
    const int64_t ldb = layout == NANOVLLM_GEMM_B_NK ? k : n;
    const int rc = nanovllm_gemm(a.data_ptr(), b.data_ptr(), out.data_ptr(), m, n, k, k, ldb, n, layout,
                                 dtype_code(a.scalar_type()), dtype_code(od), stream);
    TORCH_CHECK(rc == NANOVLLM_GEMM_OK, "nanovllm_gemm failed (code ", rc, "): ", nanovllm_gemm_last_error());
    return out;
}

at::Tensor gemm(const at::Tensor& a, const at::Tensor& w, std::optional<at::ScalarType> out_dtype) {
    return launch(a, w, out_dtype, NANOVLLM_GEMM_B_NK);
}

at::Tensor gemm_kn(const at::Tensor& a, const at::Tensor& b, std::optional<at::ScalarType> out_dtype) {
    return launch(a, b, out_dtype, NANOVLLM_GEMM_B_KN);
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(nanovllm, m) {
    m.def("gemm(Tensor a, Tensor w, ScalarType? out_dtype=None) -> Tensor");
    m.def("gemm_kn(Tensor a, Tensor b, ScalarType? out_dtype=None) -> Tensor");
}

// CUDA is the key of HIP tensors in a ROCm build of PyTorch.  The CPU key
// gets the same function so CPU operands meet the contract's message.
TORCH_LIBRARY_IMPL(nanovllm, CUDA, m) {
    m.impl("gemm", &gemm);
    m.impl("gemm_kn", &gemm_kn);
}

TORCH_LIBRARY_IMPL(nanovllm, CPU, m) {
    m.impl("gemm", &gemm);
    m.impl("gemm_kn", &gemm_kn);
}
