// PyTorch (ROCm) binding `fa._C.forward`: checks tensors, allocates O, and calls the C ABI of
// libfa_hip.so (include/fa_hip.h) on the current HIP stream of torch.
//
// Same signature, defaults and error conditions as the reference binding
// (csrc/bindings.cpp:28-73): RuntimeError with the words "CUDA", "float16", "contiguous",
// "[B, H, N, D]", "same shape", "same device" for bad tensors and "variant" for an unknown
// variant name; ValueError (std::invalid_argument) for arguments the launcher rejects, e.g.
// "head_dim must be 64 or 128". The device check says "CUDA" because torch-ROCm exposes HIP
// devices under the `cuda` device type.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/extension.h>

#include <cmath>
#include <optional>
#include <stdexcept>
#include <string>

#include "fa_hip.h"

namespace {

uint8_t parse_variant(const std::string& name) {
    if (name == "opt") return FA_VARIANT_OPT;
    if (name == "fp16acc") return FA_VARIANT_FP16ACC;
    if (name == "baseline") return FA_VARIANT_BASELINE;
    TORCH_CHECK(false, "variant must be 'opt', 'fp16acc' or 'baseline', got '", name, "'");
}

torch::Tensor forward(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                      bool causal, std::optional<double> softmax_scale,
                      const std::string& variant) {
    for (const auto* t : {&q, &k, &v}) {
        TORCH_CHECK(t->is_cuda(), "q, k, v must be CUDA (HIP) tensors");
        TORCH_CHECK(t->scalar_type() == torch::kHalf, "q, k, v must be float16");
        TORCH_CHECK(t->is_contiguous(), "q, k, v must be contiguous");
        TORCH_CHECK(t->dim() == 4, "q, k, v must have shape [B, H, N, D]");
    }
    TORCH_CHECK(q.sizes() == k.sizes() && q.sizes() == v.sizes(),
                "q, k, v must have the same shape");
    TORCH_CHECK(q.device() == k.device() && q.device() == v.device(),
                "q, k, v must be on the same device");
    const uint8_t var = parse_variant(variant);

    // torch-ROCm tags HIP devices as DeviceType::CUDA; the masquerading guard and stream
    // accessors are its HIP implementations for that device type.
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);

    const auto head_dim = q.size(3);
    fa_params p{};
    p.q = q.data_ptr();
    p.k = k.data_ptr();
    p.v = v.data_ptr();
    p.o = o.data_ptr();
    p.batch = static_cast<int32_t>(q.size(0));
    p.heads = static_cast<int32_t>(q.size(1));
    p.seqlen = static_cast<int32_t>(q.size(2));
    p.head_dim = static_cast<int32_t>(head_dim);
    // Default scale computed in double, then rounded once (csrc/bindings.cpp:55-56).
    p.softmax_scale = static_cast<float>(
        softmax_scale.value_or(1.0 / std::sqrt(static_cast<double>(head_dim))));
    p.causal = causal ? 1 : 0;
    p.variant = var;

    // N = 0 (or any empty dimension) returns an empty output without a launch
    // (csrc/bindings.cpp:60-62).
    if (q.numel() == 0) return o;
    const int rc = fa_flash_fwd(
        &p, c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.device().index()).stream());
    if (rc == FA_EINVAL) throw std::invalid_argument(fa_last_error());
    if (rc != FA_OK) throw std::runtime_error(fa_last_error());
    return o;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "FlashAttention-2 forward for MI355X (gfx950): HIP kernels behind a C ABI";
    m.def("forward", &forward, "FlashAttention forward: O = softmax(Q K^T * scale) V",
          py::arg("q"), py::arg("k"), py::arg("v"), py::arg("causal") = false,
          py::arg("softmax_scale") = py::none(), py::arg("variant") = "opt");
    m.def("version", []() { return std::string(fa_version()); });
}
