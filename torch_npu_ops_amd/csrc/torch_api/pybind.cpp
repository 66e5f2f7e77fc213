// Python module _xk_torch: the C++ drop-in API (triton_ops_api.h,
// ascendc_ops_api.h, kernel_registry.h, operation_factory.h) exposed for the
// test suite, with the reference's argument names and defaults.
#include <torch/extension.h>

#include "ascendc_ops_api.h"
#include "kernel_registry.h"
#include "operation_factory.h"
#include "triton_ops_api.h"

namespace npu = xllm::kernel::npu;
using OptT = std::optional<torch::Tensor>;

PYBIND11_MODULE(_xk_torch, m) {
  using namespace pybind11::literals;
  m.def("npu_l2norm_last_dim", &npu::npu_l2norm_last_dim, "x"_a, "eps"_a = 1e-6);
  m.def("layer_norm_fwd", &npu::layer_norm_fwd, "x"_a, "weight"_a, "bias"_a, "eps"_a,
        "z"_a = OptT(), "group_size"_a = -1, "norm_before_gate"_a = true,
        "is_rms_norm"_a = false);
  m.def("npu_split_rmsnorm_rope", &npu::npu_split_rmsnorm_rope, "input"_a, "sin"_a, "cos"_a,
        "q_weight"_a, "k_weight"_a, "q_hidden_size"_a, "kv_hidden_size"_a, "head_dim"_a, "eps"_a,
        "q_bias"_a = OptT(), "k_bias"_a = OptT(), "bias"_a = false);
  m.def("npu_causal_conv1d_update", &npu::npu_causal_conv1d_update, "x"_a, "conv_state"_a,
        "weight"_a, "activation"_a = true, "bias"_a = OptT(), "cache_seqlens"_a = OptT(),
        "conv_state_indices"_a = OptT(), "num_accepted_tokens"_a = OptT(),
        "query_start_loc"_a = OptT(), "max_query_len"_a = -1,
        "intermediate_conv_window"_a = OptT(), "pad_slot_id"_a = -1, "validate_data"_a = false);
  m.def("npu_causal_conv1d_update_v2", &npu::npu_causal_conv1d_update_v2, "x"_a, "conv_state"_a,
        "weight"_a, "activation"_a = true, "bias"_a = OptT(), "conv_state_indices"_a = OptT(),
        "query_start_loc"_a = OptT(), "max_query_len"_a = -1, "pad_slot_id"_a = -1,
        "block_idx_last_scheduled_token"_a = OptT(), "initial_state_idx"_a = OptT(),
        "validate_data"_a = false, "num_accepted_tokens"_a = OptT());
  m.def("npu_fused_recurrent_gated_delta_rule", &npu::npu_fused_recurrent_gated_delta_rule,
        "q"_a, "k"_a, "v"_a, "g"_a, "beta"_a = OptT(), "scale"_a = std::optional<float>(),
        "initial_state"_a = OptT(), "inplace_final_state"_a = true, "cu_seqlens"_a = OptT(),
        "ssm_state_indices"_a = OptT(), "num_accepted_tokens"_a = OptT(),
        "use_qk_l2norm_in_kernel"_a = false);
  m.def("rope_inplace", [](torch::Tensor x, torch::Tensor sin, torch::Tensor cos,
                           uint32_t rope_dim) {
    npu::rope_inplace(x, sin, cos, rope_dim);
    return x;
  }, "x"_a, "sin"_a, "cos"_a, "rope_dim"_a = 64);
  m.def("npu_fused_gdn_gating", &npu::npu_fused_gdn_gating, "A_log"_a, "a"_a, "b"_a,
        "dt_bias"_a, "beta"_a = 1.0f, "threshold"_a = 20.0f);
  m.def("npu_fused_sigmoid_gating_delta_rule_update",
        &npu::npu_fused_sigmoid_gating_delta_rule_update, "A_log"_a, "a"_a, "dt_bias"_a, "q"_a,
        "k"_a, "v"_a, "b"_a, "initial_state_source"_a, "initial_state_indices"_a,
        "cu_seqlens"_a, "scale"_a = std::optional<float>(), "use_qk_l2norm_in_kernel"_a = false,
        "softplus_beta"_a = 1.0f, "softplus_threshold"_a = 20.0f);
  m.def("npu_fused_qkvzba_split_reshape_cat", &npu::npu_fused_qkvzba_split_reshape_cat,
        "mixed_qkvz"_a, "mixed_ba"_a, "num_heads_qk"_a, "num_heads_v"_a, "head_qk"_a,
        "head_v"_a);
  m.def("npu_chunk_gated_delta_rule", &npu::npu_chunk_gated_delta_rule, "q"_a, "k"_a, "v"_a,
        "g"_a, "beta"_a, "scale"_a = std::optional<float>(), "initial_state"_a = OptT(),
        "output_final_state"_a = false, "cu_seqlens"_a = OptT(), "head_first"_a = false,
        "use_qk_l2norm_in_kernel"_a = false);
  m.def("npu_chunk_local_cumsum", &npu::npu_chunk_local_cumsum, "g"_a, "chunk_size"_a,
        "cu_seqlens"_a = OptT());
  m.def("npu_chunk_scaled_dot_kkt_fwd", &npu::npu_chunk_scaled_dot_kkt_fwd, "k"_a, "beta"_a,
        "g_cumsum"_a, "chunk_size"_a = 64, "cu_seqlens"_a = OptT());
  m.def("npu_solve_tril", &npu::npu_solve_tril, "A"_a, "chunk_size"_a = 64,
        "cu_seqlens"_a = OptT(), "output_dtype"_a = torch::kFloat32);
  m.def("npu_recompute_w_u_fwd", &npu::npu_recompute_w_u_fwd, "k"_a, "v"_a, "beta"_a,
        "g_cumsum"_a, "A"_a, "cu_seqlens"_a = OptT());
  m.def("npu_chunk_gated_delta_rule_fwd_h", &npu::npu_chunk_gated_delta_rule_fwd_h, "k"_a,
        "w"_a, "u"_a, "g"_a = OptT(), "initial_state"_a = OptT(), "output_final_state"_a = false,
        "chunk_size"_a = 64, "save_new_value"_a = true, "cu_seqlens"_a = OptT(),
        "chunk_offsets"_a = OptT());
  m.def("npu_chunk_fwd_o", &npu::npu_chunk_fwd_o, "q"_a, "k"_a, "v"_a, "h"_a, "g_cumsum"_a,
        "scale"_a, "chunk_size"_a = 64, "cu_seqlens"_a = OptT());
  m.def("npu_gdn_conv_decode", &npu::npu_gdn_conv_decode, "mixed_qkv"_a, "conv_state"_a,
        "conv_weight"_a, "g"_a, "beta"_a, "ssm_state"_a, "num_heads_qk"_a, "num_heads_v"_a,
        "head_k"_a = 128, "head_v"_a = 128, "scale"_a = std::optional<float>(),
        "conv_bias"_a = OptT(), "conv_state_indices"_a = OptT(), "ssm_state_indices"_a = OptT(),
        "pad_slot_id"_a = -1, "use_qk_l2norm"_a = true);
  m.def("npu_gdn_conv_sigmoid_gating_decode", &npu::npu_gdn_conv_sigmoid_gating_decode,
        "mixed_qkv"_a, "conv_state"_a, "conv_weight"_a, "A_log"_a, "a"_a, "dt_bias"_a, "b"_a,
        "ssm_state"_a, "num_heads_qk"_a, "num_heads_v"_a, "head_k"_a = 128, "head_v"_a = 128,
        "scale"_a = std::optional<float>(), "conv_bias"_a = OptT(),
        "conv_state_indices"_a = OptT(), "ssm_state_indices"_a = OptT(), "pad_slot_id"_a = -1,
        "softplus_beta"_a = 1.0f, "softplus_threshold"_a = 20.0f, "use_qk_l2norm"_a = true);
  // npu_ops (AscendC API): gemma returns (rstd, y) for its two out-params.
  m.def("npu_ops_gemma_rms_norm", [](const torch::Tensor& x, const torch::Tensor& gamma,
                                     double eps) {
    torch::Tensor rstd, y;
    npu_ops::npu_gemma_rms_norm(x, gamma, eps, rstd, y);
    return std::make_pair(rstd, y);
  });
  m.def("npu_ops_layer_norm_fwd", &npu_ops::layer_norm_fwd, "x"_a, "weight"_a, "bias"_a,
        "eps"_a, "z"_a, "group_size"_a, "norm_before_gate"_a, "is_rms_norm"_a);
  // Registry / factory shims.
  m.def("registry_register", [](const std::string& name, const std::string& path) {
    return npu::KernelRegistry::get_instance().register_kernel(name, path);
  });
  m.def("registry_stub", [](const std::string& name) {
    return reinterpret_cast<uintptr_t>(npu::KernelRegistry::get_instance().get_kernel_stub(name));
  });
  m.def("factory_kernel_name", [](const std::string& method) -> std::string {
    auto& f = npu::OperationFactory::instance();
    if (method == "layer_norm_fwd") return f.layer_norm_fwd().kernel_name();
    if (method == "chunk_fwd_o") return f.chunk_fwd_o().kernel_name();
    if (method == "split_rmsnorm_rope") return f.split_rmsnorm_rope().kernel_name();
    return "";
  });
  m.def("operation_base_paths", [](const std::string& name, std::optional<std::string> path) {
    npu::OperationBase op = path ? npu::OperationBase(name, *path) : npu::OperationBase(name);
    return std::make_pair(op.kernel_name(), op.npubin_path());
  });
  m.def("factory_status_of_invalid_layer_norm", []() {
    // execute() forwards to the C-ABI: an invalid call returns its status.
    return npu::OperationFactory::instance().layer_norm_fwd().execute(
        nullptr, 0, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr, nullptr, -1, 0, 0, 1e-5f,
        1, 0, XK_BF16, XK_BF16, nullptr);
  });
}
