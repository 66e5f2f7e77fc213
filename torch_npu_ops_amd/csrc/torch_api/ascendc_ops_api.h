// Drop-in for xLLM's ascendc_npu/ascendc_ops_api.h (namespace npu_ops): the
// same two entry points, backed by the gfx950 normalisation kernels of
// libxk.so instead of aclnnGemmaRmsNorm / aclnnLayerNormFwd.
#pragma once

#include <torch/torch.h>

#include <vector>

namespace npu_ops {

// yOut = x * rsqrt(mean(x^2) + eps) * (1 + gamma); rstdOut fp32 with x's
// leading dims followed by gamma.dim() ones (ascendc_npu/gemma_rms_norm.cpp:28-57).
void npu_gemma_rms_norm(const torch::Tensor& x, const torch::Tensor& gamma, double epsilon,
                        torch::Tensor& rstdOut, torch::Tensor& yOut);

// Grouped LayerNorm / RMSNorm with optional gate z (ascendc_npu/layer_norm_fwd.cpp:24-80).
torch::Tensor layer_norm_fwd(const torch::Tensor& x, const torch::Tensor& weight,
                             const c10::optional<torch::Tensor>& bias, double eps,
                             const c10::optional<torch::Tensor>& z, int64_t group_size,
                             bool norm_before_gate, bool is_rms_norm);

}  // namespace npu_ops
