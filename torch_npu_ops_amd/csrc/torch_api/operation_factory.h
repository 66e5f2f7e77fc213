// Compatibility shim for xLLM's triton_npu/torch_api/operation_factory.h:
// OperationFactory::instance().<op>() returns the operation object of that
// kernel (operations.h), named by the reference's kernel name.
#pragma once

#include "operations.h"

namespace xllm::kernel::npu {

class OperationFactory {
 public:
  static OperationFactory& instance() {
    static OperationFactory f;
    return f;
  }

#define XK_FACTORY(METHOD, TYPE, NAME) \
  TYPE& METHOD() {                     \
    static TYPE op(NAME);              \
    return op;                         \
  }

  XK_FACTORY(l2norm_fwd, L2NormFwdOp, "l2norm_fwd_kernel2_loop")
  XK_FACTORY(layer_norm_fwd, LayerNormFwdOp, "layer_norm_fwd_kernel")
  XK_FACTORY(layer_norm_fwd_fast, LayerNormFwdFastOp, "layer_norm_fwd_kernel_fast")
  XK_FACTORY(layer_norm_fwd_fast_rms_bias, LayerNormFwdFastRMSBiasOp,
             "layer_norm_fwd_kernel_fast_rms_bias")
  XK_FACTORY(layer_norm_fwd_fast_rms_nobias, LayerNormFwdFastRMSNoBiasOp,
             "layer_norm_fwd_kernel_fast_rms_nobias")
  XK_FACTORY(layer_norm_fwd_fast_bf16, LayerNormFwdFastBF16Op, "layer_norm_fwd_kernel_fast_bf16")
  XK_FACTORY(layer_norm_fwd_fast_rms_bf16_bias, LayerNormFwdFastRMSBF16BiasOp,
             "layer_norm_fwd_kernel_fast_rms_bf16_bias")
  XK_FACTORY(layer_norm_fwd_fast_rms_bf16_nobias, LayerNormFwdFastRMSBF16NoBiasOp,
             "layer_norm_fwd_kernel_fast_rms_bf16_nobias")
  XK_FACTORY(layer_norm_fwd_fast_z, LayerNormFwdFastZOp, "layer_norm_fwd_kernel_fast_z")
  XK_FACTORY(layer_norm_fwd_fast_rms_z_bias, LayerNormFwdFastRMSZBiasOp,
             "layer_norm_fwd_kernel_fast_rms_z_bias")
  XK_FACTORY(layer_norm_fwd_fast_rms_z_nobias, LayerNormFwdFastRMSZNoBiasOp,
             "layer_norm_fwd_kernel_fast_rms_z_nobias")
  XK_FACTORY(layer_norm_fwd_fast_bf16_z, LayerNormFwdFastBF16ZOp,
             "layer_norm_fwd_kernel_fast_bf16_z")
  XK_FACTORY(layer_norm_fwd_fast_rms_bf16_z_bias, LayerNormFwdFastRMSBF16ZBiasOp,
             "layer_norm_fwd_kernel_fast_rms_bf16_z_bias")
  XK_FACTORY(layer_norm_fwd_fast_rms_bf16_z_nobias, LayerNormFwdFastRMSBF16ZNoBiasOp,
             "layer_norm_fwd_kernel_fast_rms_bf16_z_nobias")
  XK_FACTORY(layer_norm_fwd_fast_rms_bf16_z_nobias_nomask, LayerNormFwdFastRMSBF16ZNoBiasNoMaskOp,
             "layer_norm_fwd_kernel_fast_rms_bf16_z_nobias_nomask")
  XK_FACTORY(fused_gdn_gating, FusedGdnGatingOp, "fused_gdn_gating_decode_kernel")
  XK_FACTORY(fused_sigmoid_gating_delta_rule_update, FusedSigmoidGatingDeltaRuleUpdateOp,
             "fused_sigmoid_gating_delta_rule_update_kernel")
  XK_FACTORY(recurrent_gated_delta_rule_fwd, RecurrentGatedDeltaRuleFwdOp,
             "fused_recurrent_gated_delta_rule_fwd_kernel")
  XK_FACTORY(recurrent_gated_delta_rule_spec_fwd, RecurrentGatedDeltaRuleSpecFwdOp,
             "fused_recurrent_gated_delta_rule_spec_fwd_kernel")
  XK_FACTORY(chunk_gated_delta_rule_fwd_h, ChunkGatedDeltaRuleFwdHOp,
             "chunk_gated_delta_rule_fwd_kernel_h_blockdim64")
  XK_FACTORY(chunk_local_cumsum_scalar, ChunkLocalCumsumScalarOp,
             "chunk_local_cumsum_scalar_kernel")
  XK_FACTORY(chunk_scaled_dot_kkt_fwd, ChunkScaledDotKktFwdOp, "chunk_scaled_dot_kkt_fwd_kernel")
  XK_FACTORY(solve_tril_16x16, SolveTril16x16Op, "solve_tril_16x16_kernel")
  XK_FACTORY(merge_16x16_to_64x64_inverse, Merge16x16To64x64InverseOp,
             "merge_16x16_to_64x64_inverse_kernel")
  XK_FACTORY(recompute_w_u_fwd, RecomputeWUForwardOp, "recompute_w_u_fwd_kernel")
  XK_FACTORY(chunk_fwd_o, ChunkForwardOOp, "chunk_fwd_kernel_o")
  XK_FACTORY(causal_conv1d_update_no_cache_no_mtp, CausalConv1dUpdateNoCacheNoMtpOp,
             "_causal_conv1d_update_kernel_no_cache_len_no_mtp")
  XK_FACTORY(causal_conv1d_update_qwen_decode, CausalConv1dUpdateQwenDecodeOp,
             "_causal_conv1d_update_qwen_decode_kernel")
  XK_FACTORY(causal_conv1d_update_tiled_v2, CausalConv1dUpdateTiledV2Op,
             "_causal_conv1d_update_kernel_npu_tiled_v2")
  XK_FACTORY(split_rmsnorm_rope, SplitRmsnormRopeOp, "split_rmsnorm_rope_kernel")
  XK_FACTORY(rope_inplace, RopeInplaceOp, "rope_inplace_kernel")
  XK_FACTORY(fused_qkvzba_split_reshape_gqa_r1, FusedQkvzbaSplitReshapeGqaR1Op,
             "fused_qkvzba_split_reshape_cat_gqa_r1_kernel")
  XK_FACTORY(fused_qkvzba_split_reshape_gqa_r2, FusedQkvzbaSplitReshapeGqaR2Op,
             "fused_qkvzba_split_reshape_cat_gqa_r2_kernel")
  XK_FACTORY(fused_qkvzba_split_reshape_gqa_r3, FusedQkvzbaSplitReshapeGqaR3Op,
             "fused_qkvzba_split_reshape_cat_gqa_r3_kernel")
  XK_FACTORY(fused_qkvzba_split_reshape_gqa_r4, FusedQkvzbaSplitReshapeGqaR4Op,
             "fused_qkvzba_split_reshape_cat_gqa_r4_kernel")
  XK_FACTORY(chunk_gated_delta_rule_fused, ChunkGatedDeltaRuleFusedOp, "xk_gdn_chunk_fwd")
  XK_FACTORY(gdn_conv_decode, GdnConvDecodeOp, "xk_gdn_conv_decode")

#undef XK_FACTORY

 private:
  OperationFactory() = default;
};

}  // namespace xllm::kernel::npu
