// PyTorch (ROCm) binding `fa._C`: checks tensors, allocates O (and the LSE or the split-KV
// workspace where asked), and calls the C ABI of libfa_hip.so (include/fa_hip.h) on the current
// HIP stream of torch. `forward` mirrors the reference binding; `forward_lse` and
// `forward_splitkv` are additions of this library (no reference counterpart).
//
// Grids too small to fill the GPU (few heads, long sequences): where the library's split-KV
// plan says its split path is the faster one (fa_splitkv_info.preferred), `forward` and
// `forward_lse` run it, and where fa_tail_plan plans a head split they run that (the first
// heads in one launch, the rest split-KV), with the workspace taken from torch's caching
// allocator;
// fa_flash_fwd itself stays a single allocation-free launch.
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

void check_qkv(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v) {
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
}

fa_params make_params(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                      const torch::Tensor& o, bool causal, std::optional<double> softmax_scale,
                      uint8_t variant) {
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
    p.variant = variant;
    return p;
}

void check_rc(int rc) {
    if (rc == FA_EINVAL) throw std::invalid_argument(fa_last_error());
    if (rc != FA_OK) throw std::runtime_error(fa_last_error());
}

hipStream_t stream_of(const torch::Tensor& q) {
    return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.device().index()).stream();
}

// Runs the split-KV path if the library prefers it for these params; false (nothing launched)
// otherwise, including for params the plan rejects (fa_flash_fwd then reports them).
bool splitkv_if_preferred(const fa_params& p, float* lse, const torch::Tensor& q) {
    fa_splitkv_info info{};
    if (fa_splitkv_plan(&p, 0, &info) != FA_OK || info.preferred == 0) return false;
    auto ws = torch::empty({static_cast<int64_t>(info.workspace_bytes / 4)},
                           q.options().dtype(torch::kFloat));
    check_rc(fa_flash_fwd_splitkv(&p, lse, 0, ws.data_ptr(), info.workspace_bytes, stream_of(q)));
    return true;
}

// Runs the head split of fa_tail_plan if it plans one (heads [0, h) in one launch, the rest
// through split-KV, on the same stream); false (nothing launched) otherwise.
bool tail_split_if_planned(const fa_params& p, float* lse, const torch::Tensor& q) {
    int64_t h = 0;
    if (fa_tail_plan(&p, &h) != FA_OK || h <= 0) return false;
    const int64_t bh = static_cast<int64_t>(p.batch) * p.heads;
    const int64_t head_elems = static_cast<int64_t>(p.seqlen) * p.head_dim;
    auto advance = [&](const void* ptr) {
        return static_cast<const void*>(static_cast<const at::Half*>(ptr) + h * head_elems);
    };
    fa_params first = p;
    first.batch = 1;
    first.heads = static_cast<int32_t>(h);
    fa_params rest = p;
    rest.batch = 1;
    rest.heads = static_cast<int32_t>(bh - h);
    rest.q = advance(p.q);
    rest.k = advance(p.k);
    rest.v = advance(p.v);
    rest.o = const_cast<void*>(advance(p.o));
    const hipStream_t s = stream_of(q);
    check_rc(lse ? fa_flash_fwd_lse(&first, lse, s) : fa_flash_fwd(&first, s));
    fa_splitkv_info info{};
    check_rc(fa_splitkv_plan(&rest, 0, &info));
    auto ws = torch::empty({static_cast<int64_t>(info.workspace_bytes / 4)},
                           q.options().dtype(torch::kFloat));
    check_rc(fa_flash_fwd_splitkv(&rest, lse ? lse + h * p.seqlen : nullptr, 0, ws.data_ptr(),
                                  info.workspace_bytes, s));
    return true;
}

torch::Tensor forward(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                      bool causal, std::optional<double> softmax_scale,
                      const std::string& variant) {
    check_qkv(q, k, v);
    const uint8_t var = parse_variant(variant);
    // torch-ROCm tags HIP devices as DeviceType::CUDA; the masquerading guard and stream
    // accessors are its HIP implementations for that device type.
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);
    const fa_params p = make_params(q, k, v, o, causal, softmax_scale, var);
    // N = 0 returns an empty output without a launch (csrc/bindings.cpp:60-62); any other empty
    // dimension (B, H or D = 0) reaches the launcher, which rejects it with ValueError
    // ("batch, heads and seqlen must be positive", "head_dim must be 64 or 128, got 0").
    if (q.size(2) == 0) return o;
    if (splitkv_if_preferred(p, nullptr, q)) return o;
    if (tail_split_if_planned(p, nullptr, q)) return o;
    check_rc(fa_flash_fwd(&p, stream_of(q)));
    return o;
}

// (O, LSE): LSE [B, H, N] fp32, natural log of each row's sum of exp(scale * q.k).
std::tuple<torch::Tensor, torch::Tensor> forward_lse(const torch::Tensor& q,
                                                     const torch::Tensor& k,
                                                     const torch::Tensor& v, bool causal,
                                                     std::optional<double> softmax_scale,
                                                     const std::string& variant) {
    check_qkv(q, k, v);
    const uint8_t var = parse_variant(variant);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);
    auto lse = torch::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(torch::kFloat));
    const fa_params p = make_params(q, k, v, o, causal, softmax_scale, var);
    if (q.size(2) == 0) return {o, lse};
    // Same path choice as forward, so that O is bitwise forward's.
    if (splitkv_if_preferred(p, lse.data_ptr<float>(), q)) return {o, lse};
    if (tail_split_if_planned(p, lse.data_ptr<float>(), q)) return {o, lse};
    check_rc(fa_flash_fwd_lse(&p, lse.data_ptr<float>(), stream_of(q)));
    return {o, lse};
}

// Split-KV forward (num_splits 0 = automatic); the fp32 workspace comes from torch's caching
// allocator and lives until the kernels that use it have run (stream-ordered reuse).
std::tuple<torch::Tensor, torch::Tensor> forward_splitkv(const torch::Tensor& q,
                                                         const torch::Tensor& k,
                                                         const torch::Tensor& v, bool causal,
                                                         std::optional<double> softmax_scale,
                                                         int64_t num_splits) {
    check_qkv(q, k, v);
    TORCH_CHECK(num_splits >= 0 && num_splits <= INT32_MAX, "num_splits must be >= 0");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    auto o = torch::empty_like(q);
    auto lse = torch::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(torch::kFloat));
    fa_params p = make_params(q, k, v, o, causal, softmax_scale, FA_VARIANT_OPT);
    if (q.size(2) == 0) return {o, lse};
    fa_splitkv_info info{};
    check_rc(fa_splitkv_plan(&p, static_cast<int32_t>(num_splits), &info));
    auto ws = torch::empty({static_cast<int64_t>(info.workspace_bytes / 4)},
                           q.options().dtype(torch::kFloat));
    check_rc(fa_flash_fwd_splitkv(&p, lse.data_ptr<float>(), static_cast<int32_t>(num_splits),
                                  ws.data_ptr(), info.workspace_bytes, stream_of(q)));
    return {o, lse};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "FlashAttention-2 forward for MI355X (gfx950): HIP kernels behind a C ABI";
    m.def("forward", &forward, "FlashAttention forward: O = softmax(Q K^T * scale) V",
          py::arg("q"), py::arg("k"), py::arg("v"), py::arg("causal") = false,
          py::arg("softmax_scale") = py::none(), py::arg("variant") = "opt");
    m.def("forward_lse", &forward_lse, "forward that also returns the row log-sum-exp [B, H, N]",
          py::arg("q"), py::arg("k"), py::arg("v"), py::arg("causal") = false,
          py::arg("softmax_scale") = py::none(), py::arg("variant") = "opt");
    m.def("forward_splitkv", &forward_splitkv,
          "split-KV forward for small grids; returns (O, LSE)", py::arg("q"), py::arg("k"),
          py::arg("v"), py::arg("causal") = false, py::arg("softmax_scale") = py::none(),
          py::arg("num_splits") = 0);
    m.def("version", []() { return std::string(fa_version()); });
}
