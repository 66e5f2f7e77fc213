// Torch-level C++ API of the op set, a drop-in for xLLM's
// triton_npu/torch_api/triton_ops_api.h (namespace xllm::kernel::npu): the
// same function names, argument lists and defaults for the hot-path ops, on
// PyTorch-ROCm tensors.  Each function validates with TORCH_CHECK, allocates
// its outputs on the input's device, and launches the gfx950 kernels of
// libxk.so (include/xk_ops.h) on the current HIP stream.
//
// Differences from the reference, all deliberate:
//  * a failed launch throws (c10::Error) instead of being logged;
//  * none on the flags the reference binaries bake in: as there,
//    npu_causal_conv1d_update always applies SiLU (`activation` is ignored)
//    and the recurrent and sigmoid-gating GDN ops always l2-normalise q and
//    k (`use_qk_l2norm_in_kernel` is ignored); the C-ABI keeps both switches;
//  * fp32 inputs are accepted where the reference binaries were bf16-only
//    (split_rmsnorm_rope, l2norm);
//  * the chunked op runs its whole pipeline on the device without reading
//    cu_seqlens on the host.
#pragma once

#include <torch/torch.h>

#include <optional>
#include <tuple>
#include <utility>

namespace xllm::kernel::npu {

torch::Tensor npu_l2norm_last_dim(torch::Tensor& x, double eps = 1e-6);

// Chunk gated delta rule pipeline operators
torch::Tensor npu_chunk_local_cumsum(const torch::Tensor& g, int64_t chunk_size,
                                     const std::optional<torch::Tensor>& cu_seqlens);

torch::Tensor npu_chunk_scaled_dot_kkt_fwd(const torch::Tensor& k, const torch::Tensor& beta,
                                           const torch::Tensor& g_cumsum, int64_t chunk_size,
                                           const std::optional<torch::Tensor>& cu_seqlens);

torch::Tensor npu_solve_tril(const torch::Tensor& A, int64_t chunk_size,
                             const std::optional<torch::Tensor>& cu_seqlens,
                             torch::ScalarType output_dtype);

std::pair<torch::Tensor, torch::Tensor> npu_recompute_w_u_fwd(
    const torch::Tensor& k, const torch::Tensor& v, const torch::Tensor& beta,
    const torch::Tensor& g_cumsum, const torch::Tensor& A,
    const std::optional<torch::Tensor>& cu_seqlens);

torch::Tensor npu_chunk_fwd_o(const torch::Tensor& q, const torch::Tensor& k,
                              const torch::Tensor& v, const torch::Tensor& h,
                              const torch::Tensor& g_cumsum, float scale, int64_t chunk_size,
                              const std::optional<torch::Tensor>& cu_seqlens);

void rope_inplace(torch::Tensor& x, torch::Tensor& sin, torch::Tensor& cos,
                  uint32_t rope_dim = 64);

std::pair<torch::Tensor, torch::Tensor> npu_fused_gdn_gating(torch::Tensor& A_log,
                                                             torch::Tensor& a, torch::Tensor& b,
                                                             torch::Tensor& dt_bias,
                                                             float beta = 1.0f,
                                                             float threshold = 20.0f);

std::pair<torch::Tensor, torch::Tensor> npu_fused_recurrent_gated_delta_rule(
    torch::Tensor& q, torch::Tensor& k, torch::Tensor& v, torch::Tensor& g,
    const std::optional<torch::Tensor>& beta = std::nullopt,
    const std::optional<float>& scale = std::nullopt,
    const std::optional<torch::Tensor>& initial_state = std::nullopt,
    bool inplace_final_state = true,
    const std::optional<torch::Tensor>& cu_seqlens = std::nullopt,
    const std::optional<torch::Tensor>& ssm_state_indices = std::nullopt,
    const std::optional<torch::Tensor>& num_accepted_tokens = std::nullopt,
    bool use_qk_l2norm_in_kernel = false);

torch::Tensor npu_fused_sigmoid_gating_delta_rule_update(
    torch::Tensor& A_log, torch::Tensor& a, torch::Tensor& dt_bias, torch::Tensor& q,
    torch::Tensor& k, torch::Tensor& v, torch::Tensor& b, torch::Tensor& initial_state_source,
    torch::Tensor& initial_state_indices, torch::Tensor& cu_seqlens,
    const std::optional<float>& scale = std::nullopt, bool use_qk_l2norm_in_kernel = false,
    float softplus_beta = 1.0f, float softplus_threshold = 20.0f);

std::pair<torch::Tensor, torch::Tensor> npu_chunk_gated_delta_rule(
    torch::Tensor& q, torch::Tensor& k, torch::Tensor& v, torch::Tensor& g, torch::Tensor& beta,
    const std::optional<float>& scale = std::nullopt,
    const std::optional<torch::Tensor>& initial_state = std::nullopt,
    bool output_final_state = false,
    const std::optional<torch::Tensor>& cu_seqlens = std::nullopt, bool head_first = false,
    bool use_qk_l2norm_in_kernel = false);

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> npu_chunk_gated_delta_rule_fwd_h(
    torch::Tensor& k, torch::Tensor& w, torch::Tensor& u,
    const std::optional<torch::Tensor>& g = std::nullopt,
    const std::optional<torch::Tensor>& initial_state = std::nullopt,
    bool output_final_state = false, int64_t chunk_size = 64, bool save_new_value = true,
    const std::optional<torch::Tensor>& cu_seqlens = std::nullopt,
    const std::optional<torch::Tensor>& chunk_offsets = std::nullopt);

torch::Tensor layer_norm_fwd(torch::Tensor& x, torch::Tensor& weight, torch::Tensor& bias,
                             double eps, const std::optional<torch::Tensor>& z = std::nullopt,
                             int64_t group_size = -1, bool norm_before_gate = true,
                             bool is_rms_norm = false);

torch::Tensor npu_causal_conv1d_update(
    torch::Tensor& x, torch::Tensor& conv_state, torch::Tensor& weight, bool activation = true,
    const std::optional<torch::Tensor>& bias = std::nullopt,
    const std::optional<torch::Tensor>& cache_seqlens = std::nullopt,
    const std::optional<torch::Tensor>& conv_state_indices = std::nullopt,
    const std::optional<torch::Tensor>& num_accepted_tokens = std::nullopt,
    const std::optional<torch::Tensor>& query_start_loc = std::nullopt,
    int32_t max_query_len = -1,
    const std::optional<torch::Tensor>& intermediate_conv_window = std::nullopt,
    int32_t pad_slot_id = -1, bool validate_data = false);

torch::Tensor npu_causal_conv1d_update_v2(
    torch::Tensor& x, torch::Tensor& conv_state, torch::Tensor& weight, bool activation = true,
    const std::optional<torch::Tensor>& bias = std::nullopt,
    const std::optional<torch::Tensor>& conv_state_indices = std::nullopt,
    const std::optional<torch::Tensor>& query_start_loc = std::nullopt,
    int32_t max_query_len = -1, int32_t pad_slot_id = -1,
    const std::optional<torch::Tensor>& block_idx_last_scheduled_token = std::nullopt,
    const std::optional<torch::Tensor>& initial_state_idx = std::nullopt,
    bool validate_data = false,
    const std::optional<torch::Tensor>& num_accepted_tokens = std::nullopt);

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor>
npu_fused_qkvzba_split_reshape_cat(torch::Tensor& mixed_qkvz, torch::Tensor& mixed_ba,
                                   int32_t num_heads_qk, int32_t num_heads_v, int32_t head_qk,
                                   int32_t head_v);

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> npu_split_rmsnorm_rope(
    torch::Tensor& input, torch::Tensor& sin, torch::Tensor& cos, torch::Tensor& q_weight,
    torch::Tensor& k_weight, int64_t q_hidden_size, int64_t kv_hidden_size, int64_t head_dim,
    double eps, const std::optional<torch::Tensor>& q_bias = std::nullopt,
    const std::optional<torch::Tensor>& k_bias = std::nullopt, bool bias = false);

// Additions of this build (no single reference function): one decode step
// of conv1d update + SiLU, q/k/v split, l2norm and the gated delta rule on
// mixed_qkv [B, 2*Hqk*K + Hv*V]; conv_state and ssm_state are updated in
// place.  Returns o [B, Hv, V].
torch::Tensor npu_gdn_conv_decode(
    torch::Tensor& mixed_qkv, torch::Tensor& conv_state, torch::Tensor& conv_weight,
    torch::Tensor& g, const std::optional<torch::Tensor>& beta, torch::Tensor& ssm_state,
    int64_t num_heads_qk, int64_t num_heads_v, int64_t head_k = 128, int64_t head_v = 128,
    const std::optional<float>& scale = std::nullopt,
    const std::optional<torch::Tensor>& conv_bias = std::nullopt,
    const std::optional<torch::Tensor>& conv_state_indices = std::nullopt,
    const std::optional<torch::Tensor>& ssm_state_indices = std::nullopt,
    int32_t pad_slot_id = -1, bool use_qk_l2norm = true);

// The same decode step with the gating in the kernel: g = -exp(A_log) *
// softplus(a + dt_bias) and beta = sigmoid(b) per (row, v head), as
// npu_fused_sigmoid_gating_delta_rule_update forms them; a, b [B, Hv],
// A_log, dt_bias fp32 [Hv].  One launch from the projection outputs.
torch::Tensor npu_gdn_conv_sigmoid_gating_decode(
    torch::Tensor& mixed_qkv, torch::Tensor& conv_state, torch::Tensor& conv_weight,
    torch::Tensor& A_log, torch::Tensor& a, torch::Tensor& dt_bias, torch::Tensor& b,
    torch::Tensor& ssm_state, int64_t num_heads_qk, int64_t num_heads_v, int64_t head_k = 128,
    int64_t head_v = 128, const std::optional<float>& scale = std::nullopt,
    const std::optional<torch::Tensor>& conv_bias = std::nullopt,
    const std::optional<torch::Tensor>& conv_state_indices = std::nullopt,
    const std::optional<torch::Tensor>& ssm_state_indices = std::nullopt,
    int32_t pad_slot_id = -1, float softplus_beta = 1.0f, float softplus_threshold = 20.0f,
    bool use_qk_l2norm = true);

}  // namespace xllm::kernel::npu
