// KernelRegistry over the kernels built into libxk.so (kernel_registry.h).
#include "kernel_registry.h"

#include <cstring>

#include "xk_ops.h"

namespace xllm::kernel::npu {
namespace {

struct Entry {
  const char* name;
  void* stub;
};

// The reference's kernel names (triton_npu/torch_api/operation_factory.h)
// of the ops this build provides, with the entry point that runs each.
const Entry kKernels[] = {
    {"l2norm_fwd_kernel2_loop", reinterpret_cast<void*>(&xk_l2norm_last_dim)},
    {"layer_norm_fwd_kernel", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_bias", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_nobias", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_bf16", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_bf16_bias", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_bf16_nobias", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_z", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_z_bias", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_z_nobias", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_bf16_z", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_bf16_z_bias", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_bf16_z_nobias", reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"layer_norm_fwd_kernel_fast_rms_bf16_z_nobias_nomask",
     reinterpret_cast<void*>(&xk_layer_norm_fwd)},
    {"fused_gdn_gating_decode_kernel", reinterpret_cast<void*>(&xk_fused_gdn_gating)},
    {"fused_sigmoid_gating_delta_rule_update_kernel",
     reinterpret_cast<void*>(&xk_gdn_sigmoid_gating_update)},
    {"fused_recurrent_gated_delta_rule_fwd_kernel", reinterpret_cast<void*>(&xk_gdn_recurrent)},
    {"fused_recurrent_gated_delta_rule_spec_fwd_kernel",
     reinterpret_cast<void*>(&xk_gdn_recurrent)},
    {"chunk_gated_delta_rule_fwd_kernel_h_blockdim64", reinterpret_cast<void*>(&xk_chunk_fwd_h)},
    {"chunk_local_cumsum_scalar_kernel", reinterpret_cast<void*>(&xk_chunk_local_cumsum)},
    {"chunk_scaled_dot_kkt_fwd_kernel", reinterpret_cast<void*>(&xk_chunk_scaled_dot_kkt)},
    {"solve_tril_16x16_kernel", reinterpret_cast<void*>(&xk_solve_tril)},
    {"merge_16x16_to_64x64_inverse_kernel", reinterpret_cast<void*>(&xk_solve_tril)},
    {"recompute_w_u_fwd_kernel", reinterpret_cast<void*>(&xk_recompute_w_u)},
    {"chunk_fwd_kernel_o", reinterpret_cast<void*>(&xk_chunk_fwd_o)},
    {"_causal_conv1d_update_kernel_no_cache_len_no_mtp",
     reinterpret_cast<void*>(&xk_causal_conv1d_update)},
    {"_causal_conv1d_update_qwen_decode_kernel", reinterpret_cast<void*>(&xk_causal_conv1d_update)},
    {"_causal_conv1d_update_kernel_npu_tiled_v2", reinterpret_cast<void*>(&xk_causal_conv1d_varlen)},
    {"split_rmsnorm_rope_kernel", reinterpret_cast<void*>(&xk_split_rmsnorm_rope)},
    {"rope_inplace_kernel", reinterpret_cast<void*>(&xk_rope_inplace)},
    {"fused_qkvzba_split_reshape_cat_gqa_r1_kernel",
     reinterpret_cast<void*>(&xk_fused_qkvzba_split_reshape_cat)},
    {"fused_qkvzba_split_reshape_cat_gqa_r2_kernel",
     reinterpret_cast<void*>(&xk_fused_qkvzba_split_reshape_cat)},
    {"fused_qkvzba_split_reshape_cat_gqa_r3_kernel",
     reinterpret_cast<void*>(&xk_fused_qkvzba_split_reshape_cat)},
    {"fused_qkvzba_split_reshape_cat_gqa_r4_kernel",
     reinterpret_cast<void*>(&xk_fused_qkvzba_split_reshape_cat)},
};

const Entry* find(const std::string& name) {
  for (const Entry& e : kKernels)
    if (name == e.name) return &e;
  return nullptr;
}

}  // namespace

KernelRegistry& KernelRegistry::get_instance() {
  static KernelRegistry r;
  return r;
}

bool KernelRegistry::register_kernel(const std::string& kernel_name,
                                     const std::string& /*binary_path*/) {
  return find(kernel_name) != nullptr;
}

KernelStubHandle KernelRegistry::get_kernel_stub(const std::string& kernel_name) const {
  const Entry* e = find(kernel_name);
  return e ? e->stub : nullptr;
}

bool KernelRegistry::is_kernel_registered(const std::string& kernel_name) const {
  return find(kernel_name) != nullptr;
}

void KernelRegistry::cleanup() {}

bool KernelRegistry::parse_json_config(const std::string& /*json_path*/, std::string& /*name*/,
                                       std::string& /*mix_mode*/, int64_t& /*workspace_size*/,
                                       int64_t& /*lock_init_value*/, int64_t& /*lock_num*/) {
  return false;
}

bool KernelRegistry::get_kernel_workspace_config(const std::string& kernel_name,
                                                 int64_t& workspace_size,
                                                 int64_t& lock_init_value,
                                                 int64_t& lock_num) const {
  if (!find(kernel_name)) return false;
  workspace_size = 0;
  lock_init_value = 0;
  lock_num = 0;
  return true;
}

}  // namespace xllm::kernel::npu
