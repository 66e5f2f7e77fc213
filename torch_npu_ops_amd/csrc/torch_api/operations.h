// Compatibility shim for xLLM's triton_npu/operations.h and
// operation_base.h: the same per-kernel operation class names, each bound to
// the xk_* C-ABI entry point that runs it.  The reference's
// execute(stream, gx, gy, gz, BuildArgsFn) packed a Triton argument blob for
// an AOT binary; here execute(args...) forwards the C-ABI arguments of that
// entry point (the stream is its last argument) and returns its status
// (XK_OK = 0).  ArgsBuilder and the binary loader have no counterpart.
#pragma once

#include <string>
#include <utility>

#include "xk_ops.h"

namespace xllm::kernel::npu {

class OperationBase {
 public:
  // npubin_path is kept for source compatibility (operation_base.h:130-133);
  // the kernels are linked in, so it only reports what the caller passed.
  explicit OperationBase(std::string kernel_name, std::string npubin_path = "")
      : kernel_name_(std::move(kernel_name)), npubin_path_(std::move(npubin_path)) {}
  virtual ~OperationBase() = default;
  const std::string& kernel_name() const { return kernel_name_; }
  const std::string& npubin_path() const { return npubin_path_; }
  // Built-in kernels are always available.
  bool is_registered() const { return true; }

 private:
  std::string kernel_name_;
  std::string npubin_path_;
};

template <auto Fn>
class XkOperation : public OperationBase {
 public:
  using OperationBase::OperationBase;
  template <typename... A>
  int execute(A&&... args) const {
    return Fn(std::forward<A>(args)...);
  }
};

#define XK_OPERATION(NAME, FN)                   \
  class NAME final : public XkOperation<&FN> {   \
   public:                                       \
    using XkOperation<&FN>::XkOperation;         \
  }

XK_OPERATION(L2NormFwdOp, xk_l2norm_last_dim);
XK_OPERATION(LayerNormFwdOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSBiasOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSNoBiasOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastBF16Op, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSBF16BiasOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSBF16NoBiasOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastZOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSZBiasOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSZNoBiasOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastBF16ZOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSBF16ZBiasOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSBF16ZNoBiasOp, xk_layer_norm_fwd);
XK_OPERATION(LayerNormFwdFastRMSBF16ZNoBiasNoMaskOp, xk_layer_norm_fwd);
XK_OPERATION(FusedGdnGatingOp, xk_fused_gdn_gating);
XK_OPERATION(RecurrentGatedDeltaRuleFwdOp, xk_gdn_recurrent);
XK_OPERATION(FusedSigmoidGatingDeltaRuleUpdateOp, xk_gdn_sigmoid_gating_update);
XK_OPERATION(RecurrentGatedDeltaRuleSpecFwdOp, xk_gdn_recurrent);
XK_OPERATION(ChunkGatedDeltaRuleFwdHOp, xk_chunk_fwd_h);
XK_OPERATION(ChunkLocalCumsumScalarOp, xk_chunk_local_cumsum);
XK_OPERATION(ChunkScaledDotKktFwdOp, xk_chunk_scaled_dot_kkt);
XK_OPERATION(SolveTril16x16Op, xk_solve_tril);
XK_OPERATION(Merge16x16To64x64InverseOp, xk_solve_tril);
XK_OPERATION(RecomputeWUForwardOp, xk_recompute_w_u);
XK_OPERATION(ChunkForwardOOp, xk_chunk_fwd_o);
XK_OPERATION(CausalConv1dUpdateNoCacheNoMtpOp, xk_causal_conv1d_update);
XK_OPERATION(CausalConv1dUpdateQwenDecodeOp, xk_causal_conv1d_update);
XK_OPERATION(CausalConv1dUpdateTiledV2Op, xk_causal_conv1d_varlen);
XK_OPERATION(SplitRmsnormRopeOp, xk_split_rmsnorm_rope);
XK_OPERATION(RopeInplaceOp, xk_rope_inplace);
XK_OPERATION(FusedQkvzbaSplitReshapeGqaR1Op, xk_fused_qkvzba_split_reshape_cat);
XK_OPERATION(FusedQkvzbaSplitReshapeGqaR2Op, xk_fused_qkvzba_split_reshape_cat);
XK_OPERATION(FusedQkvzbaSplitReshapeGqaR3Op, xk_fused_qkvzba_split_reshape_cat);
XK_OPERATION(FusedQkvzbaSplitReshapeGqaR4Op, xk_fused_qkvzba_split_reshape_cat);
// No reference counterpart: the whole chunked pipeline and the fused decode step.
XK_OPERATION(ChunkGatedDeltaRuleFusedOp, xk_gdn_chunk_fwd);
XK_OPERATION(GdnConvDecodeOp, xk_gdn_conv_decode);

#undef XK_OPERATION

}  // namespace xllm::kernel::npu
