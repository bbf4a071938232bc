// Thin libtorch shim over the W4A16 C ABI: registers the torch ops
// w4a16::linear and w4a16::dequantize with the schemas of reference
// csrc/int4_linear.cpp:16-23, implemented on the CUDA dispatch key (which is
// the HIP device on PyTorch-ROCm), and exposes an empty Python module so that
// importing the extension registers the ops (reference csrc/int4_linear.cpp:30).
//
// Tensor-level checks use the reference's messages (reference
// csrc/int4_linear_kernel.cu:646-691, :809-841); shape relations and launches
// go through the C ABI. The output comes from the caching allocator on the
// activations' device and the work is enqueued on the current stream, so the
// op is graph-capture safe.
#include <Python.h>

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "w4a16_hip.h"

namespace {

void* current_stream(const at::Device& device) {
    return static_cast<void*>(c10::hip::getCurrentHIPStream(device.index()).stream());
}

at::Tensor linear(const at::Tensor& activations, const at::Tensor& packed_weights, const at::Tensor& scales,
                  int64_t group_size) {
    TORCH_CHECK(activations.is_cuda(), "activations must be a CUDA tensor");
    TORCH_CHECK(packed_weights.is_cuda(), "packed_weights must be a CUDA tensor");
    TORCH_CHECK(scales.is_cuda(), "scales must be a CUDA tensor");
    TORCH_CHECK(activations.device() == packed_weights.device() && activations.device() == scales.device(),
                "all inputs must be on the same CUDA device");
    TORCH_CHECK(activations.scalar_type() == at::kHalf, "activations must have dtype torch.float16");
    TORCH_CHECK(packed_weights.scalar_type() == at::kByte, "packed_weights must have dtype torch.uint8");
    TORCH_CHECK(scales.scalar_type() == at::kHalf, "scales must have dtype torch.float16");
    TORCH_CHECK(activations.dim() == 2, "activations must have shape [M, K]");
    TORCH_CHECK(packed_weights.dim() == 2, "packed_weights must have shape [N, K / 2]");
    TORCH_CHECK(scales.dim() == 2, "scales must have shape [N, K / group_size]");
    TORCH_CHECK(activations.is_contiguous(), "activations must be contiguous");
    TORCH_CHECK(packed_weights.is_contiguous(), "packed_weights must be contiguous");
    TORCH_CHECK(scales.is_contiguous(), "scales must be contiguous");

    int rc = w4a16_check_linear_shapes(activations.size(0), activations.size(1), packed_weights.size(0),
                                       packed_weights.size(1), scales.size(0), scales.size(1), group_size);
    TORCH_CHECK(rc == W4A16_OK, w4a16_last_error());

    const int64_t M = activations.size(0);
    const int64_t K = activations.size(1);
    const int64_t N = packed_weights.size(0);
    const c10::DeviceGuard guard(activations.device());
    at::Tensor output = at::empty({M, N}, activations.options());
    if (M * N == 0) return output;

    // partial sums of the split-K kernel, from the caching allocator (so the
    // op stays graph-capture safe)
    const int64_t ws_bytes = w4a16_linear_workspace_bytes(M, N, K, group_size);
    at::Tensor workspace;
    if (ws_bytes > 0) workspace = at::empty({(ws_bytes + 3) / 4}, activations.options().dtype(at::kFloat));
    rc = w4a16_linear_ws_f16(activations.data_ptr(), packed_weights.data_ptr<uint8_t>(), scales.data_ptr(),
                             output.data_ptr(), M, N, K, group_size, ws_bytes > 0 ? workspace.data_ptr() : nullptr,
                             ws_bytes, current_stream(activations.device()));
    TORCH_CHECK(rc == W4A16_OK, w4a16_last_error());
    return output;
}

at::Tensor dequantize(const at::Tensor& packed_weights, const at::Tensor& scales, int64_t group_size) {
    TORCH_CHECK(packed_weights.is_cuda(), "packed_weights must be a CUDA tensor");
    TORCH_CHECK(scales.is_cuda(), "scales must be a CUDA tensor");
    TORCH_CHECK(packed_weights.device() == scales.device(),
                "packed_weights and scales must be on the same CUDA device");
    TORCH_CHECK(packed_weights.scalar_type() == at::kByte, "packed_weights must have dtype torch.uint8");
    TORCH_CHECK(scales.scalar_type() == at::kHalf, "scales must have dtype torch.float16");
    TORCH_CHECK(packed_weights.dim() == 2, "packed_weights must have shape [N, K / 2]");
    TORCH_CHECK(scales.dim() == 2, "scales must have shape [N, K / group_size]");
    TORCH_CHECK(packed_weights.is_contiguous(), "packed_weights must be contiguous");
    TORCH_CHECK(scales.is_contiguous(), "scales must be contiguous");

    int rc = w4a16_check_dequantize_shapes(packed_weights.size(0), packed_weights.size(1), scales.size(0),
                                           scales.size(1), group_size,
                                           reinterpret_cast<uint64_t>(packed_weights.data_ptr()));
    TORCH_CHECK(rc == W4A16_OK, w4a16_last_error());

    const int64_t N = packed_weights.size(0);
    const int64_t K = packed_weights.size(1) * 2;
    const c10::DeviceGuard guard(packed_weights.device());
    at::Tensor weights = at::empty({N, K}, packed_weights.options().dtype(at::kHalf));
    if (N * K == 0) return weights;
    rc = w4a16_dequantize_f16(packed_weights.data_ptr<uint8_t>(), scales.data_ptr(), weights.data_ptr(), N, K,
                              group_size, current_stream(packed_weights.device()));
    TORCH_CHECK(rc == W4A16_OK, w4a16_last_error());
    return weights;
}

}  // namespace

TORCH_LIBRARY(w4a16, m) {
    m.def("linear(Tensor activations, Tensor packed_weights, Tensor scales, int group_size) -> Tensor");
    m.def("dequantize(Tensor packed_weights, Tensor scales, int group_size) -> Tensor");
}

TORCH_LIBRARY_IMPL(w4a16, CUDA, m) {
    m.impl("linear", &linear);
    m.impl("dequantize", &dequantize);
}

static PyModuleDef w4a16_module = {PyModuleDef_HEAD_INIT, "_C", "W4A16 torch ops (registered on import)", -1,
                                   nullptr};

PyMODINIT_FUNC PyInit__C(void) { return PyModule_Create(&w4a16_module); }
