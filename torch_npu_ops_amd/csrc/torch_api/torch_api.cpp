// Implementation of triton_ops_api.h / ascendc_ops_api.h over the C-ABI of
// libxk.so.  Each function follows the reference wrapper cited beside it
// (validation, output allocation, in-place state), then calls one xk_*
// entry point on the current HIP stream and turns a non-zero status into a
// c10::Error.
#include "ascendc_ops_api.h"
#include "triton_ops_api.h"

#include <c10/hip/HIPStream.h>

#include <cmath>

#include "xk_ops.h"

namespace {

xk_dtype xdt(const torch::Tensor& t) {
  switch (t.scalar_type()) {
    case torch::kFloat32: return XK_F32;
    case torch::kBFloat16: return XK_BF16;
    case torch::kFloat16: return XK_F16;
    case torch::kInt32: return XK_I32;
    case torch::kInt64: return XK_I64;
    default: TORCH_CHECK(false, "unsupported dtype ", t.scalar_type());
  }
  return XK_F32;
}

void* stream_of(const torch::Tensor& t) {
  TORCH_CHECK(t.is_cuda(), "torch_npu_ops_amd ops need tensors on a GPU device");
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check(int st, const char* what) {
  TORCH_CHECK(st == XK_OK, what, " failed: ", xk_status_string(st), " (", st, ")");
}

template <typename T>
const void* ptr(const std::optional<T>& t) {
  return t.has_value() && t->defined() ? t->data_ptr() : nullptr;
}
const void* ptr(const torch::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }
void* mptr(torch::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

bool has(const std::optional<torch::Tensor>& t) { return t.has_value() && t->defined(); }

// Row-contiguous 2-D view of x as [-1, N].
torch::Tensor rows(const torch::Tensor& x, int64_t N) {
  auto x2 = x.reshape({-1, N});
  return x2.stride(-1) == 1 ? x2 : x2.contiguous();
}

// x as [rows, -1] with unit column stride (a copy only if needed).
torch::Tensor rows_of(const torch::Tensor& x, int64_t rows) {
  auto x2 = x.reshape({rows, -1});
  return x2.stride(-1) == 1 ? x2 : x2.contiguous();
}

// cu_seqlens on the device (int32/int64 kept), or B sequences of T tokens.
std::pair<torch::Tensor, int64_t> seqs(int64_t B, int64_t T,
                                       const std::optional<torch::Tensor>& cu_seqlens,
                                       const torch::Device& dev) {
  if (!has(cu_seqlens)) {
    return {torch::arange(0, (B + 1) * T, T, torch::TensorOptions().dtype(torch::kInt32).device(dev)),
            B};
  }
  auto cu = cu_seqlens->to(dev).contiguous();
  if (cu.scalar_type() != torch::kInt32 && cu.scalar_type() != torch::kInt64)
    cu = cu.to(torch::kInt32);
  return {cu, cu.numel() - 1};
}

// Total chunks of all sequences with the kernels' clamping of cu_seqlens
// (a host read, as the reference's infer_total_chunks,
// npu_triton_chunk_gated_delta_rule.cpp:116-138).
int64_t num_chunks(const torch::Tensor& cu, int64_t total) {
  auto c = cu.to(torch::kCPU, torch::kInt64).clamp(0, total);
  auto lens = (c.slice(0, 1) - c.slice(0, 0, -1)).clamp_min(0);
  return ((lens + 63).div(64, "floor")).sum().item<int64_t>();
}

torch::Tensor workspace(int64_t bytes, const torch::Device& dev) {
  return torch::empty({std::max<int64_t>(bytes, 1)},
                      torch::TensorOptions().dtype(torch::kUInt8).device(dev));
}

torch::Tensor layer_norm_impl(const torch::Tensor& x, const torch::Tensor& weight,
                              const torch::Tensor& bias, double eps,
                              const std::optional<torch::Tensor>& z, int64_t group_size,
                              bool norm_before_gate, bool is_rms_norm) {
  TORCH_CHECK(x.dim() >= 1, "layer_norm_fwd expects x.dim() >= 1");
  const int64_t N = x.size(-1);
  const int64_t G = group_size > 0 ? group_size : N;
  TORCH_CHECK(N % G == 0, "x.size(-1) must be divisible by group_size");
  TORCH_CHECK(weight.defined() && weight.numel() == N, "weight numel must equal x.size(-1)");
  auto x2 = rows(x, N);
  torch::Tensor z2;
  if (has(z)) {
    TORCH_CHECK(z->sizes() == x.sizes(), "z shape must match x shape");
    z2 = rows(*z, N);
  }
  const int64_t M = x2.size(0);
  auto w = weight.contiguous();
  torch::Tensor b;
  if (bias.defined() && bias.numel() > 0) {  // undefined or empty: no bias
    TORCH_CHECK(bias.numel() == N, "bias numel must equal x.size(-1)");
    b = bias.contiguous().to(w.scalar_type());
  }
  auto y = torch::empty({M, N}, x.options());
  const int64_t ng = N / G;
  // mean / rstd are allocated as the reference does (and not returned).
  auto f32 = x.options().dtype(torch::kFloat32);
  torch::Tensor mean = is_rms_norm ? torch::Tensor() : torch::empty({ng * M}, f32);
  auto rstd = torch::empty({ng * M}, f32);
  check(xk_layer_norm_fwd(x2.data_ptr(), x2.stride(0), y.data_ptr(), y.stride(0), w.data_ptr(),
                          ptr(b), ptr(z2), z2.defined() ? z2.stride(0) : 0,
                          static_cast<float*>(mptr(mean)), static_cast<float*>(rstd.data_ptr()),
                          M, N, G, static_cast<float>(eps), norm_before_gate,
                          is_rms_norm, xdt(x), xdt(w), stream_of(x)),
        "xk_layer_norm_fwd");
  return y.reshape(x.sizes());
}

}  // namespace

namespace xllm::kernel::npu {

// triton_npu/torch_api/npu_triton_l2norm.cpp:60-109
torch::Tensor npu_l2norm_last_dim(torch::Tensor& x, double eps) {
  TORCH_CHECK(x.dim() >= 1 && x.size(-1) > 0, "npu_l2norm_last_dim expects hidden dim > 0");
  auto xc = x.contiguous();
  auto y = torch::empty_like(xc);
  const int64_t cols = x.size(-1);
  check(xk_l2norm_last_dim(xc.data_ptr(), y.data_ptr(), xc.numel() / cols, cols,
                           static_cast<float>(eps), xdt(xc), xdt(y), stream_of(x)),
        "xk_l2norm_last_dim");
  return y;
}

// triton_npu/torch_api/npu_triton_layernorm_fwd.cpp:48-332
torch::Tensor layer_norm_fwd(torch::Tensor& x, torch::Tensor& weight, torch::Tensor& bias,
                             double eps, const std::optional<torch::Tensor>& z,
                             int64_t group_size, bool norm_before_gate, bool is_rms_norm) {
  return layer_norm_impl(x, weight, bias, eps, z, group_size, norm_before_gate, is_rms_norm);
}

// triton_npu/torch_api/npu_triton_split_rmsnorm_rope.cpp:56-144
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> npu_split_rmsnorm_rope(
    torch::Tensor& input, torch::Tensor& sin, torch::Tensor& cos, torch::Tensor& q_weight,
    torch::Tensor& k_weight, int64_t q_hidden_size, int64_t kv_hidden_size, int64_t head_dim,
    double eps, const std::optional<torch::Tensor>& q_bias,
    const std::optional<torch::Tensor>& k_bias, bool bias) {
  TORCH_CHECK(input.dim() == 2, "split_rmsnorm_rope input must be a 2D tensor");
  TORCH_CHECK(head_dim > 0 && (head_dim & (head_dim - 1)) == 0,
              "split_rmsnorm_rope head_dim must be a power of two");
  TORCH_CHECK(kv_hidden_size > 0 && q_hidden_size % kv_hidden_size == 0,
              "split_rmsnorm_rope q_hidden_size must be divisible by kv_hidden_size");
  TORCH_CHECK(kv_hidden_size % head_dim == 0,
              "split_rmsnorm_rope kv_hidden_size must be divisible by head_dim");
  TORCH_CHECK(input.size(1) == q_hidden_size + 2 * kv_hidden_size,
              "split_rmsnorm_rope input hidden size mismatch");
  TORCH_CHECK(q_weight.numel() == head_dim && k_weight.numel() == head_dim,
              "split_rmsnorm_rope q/k weight shape mismatch");
  const int64_t T = input.size(0);
  TORCH_CHECK(sin.dim() == 2 && cos.dim() == 2 && sin.size(0) == T && cos.size(0) == T &&
                  sin.size(1) == head_dim && cos.size(1) == head_dim,
              "split_rmsnorm_rope sin/cos shape mismatch");
  auto x = input.stride(1) == 1 ? input : input.contiguous();
  const auto aux = q_weight.scalar_type();
  auto qw = q_weight.contiguous();
  auto kw = k_weight.contiguous().to(aux);
  torch::Tensor qb, kb;
  if (bias && has(q_bias) && has(k_bias)) {  // reference :109-118
    qb = q_bias->contiguous().to(aux);
    kb = k_bias->contiguous().to(aux);
  }
  auto s = sin.to(aux).contiguous();
  auto c = cos.to(aux).contiguous();
  auto q = torch::empty({T, q_hidden_size}, input.options());
  auto k = torch::empty({T, kv_hidden_size}, input.options());
  auto v = torch::empty({T, kv_hidden_size}, input.options());
  check(xk_split_rmsnorm_rope(x.data_ptr(), x.stride(0), T, s.data_ptr(), c.data_ptr(), head_dim,
                              nullptr, XK_I64, nullptr, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                              qw.data_ptr(), ptr(qb), kw.data_ptr(), ptr(kb), xdt(qw),
                              q_hidden_size, kv_hidden_size, head_dim, static_cast<float>(eps),
                              xdt(x), stream_of(input)),
        "xk_split_rmsnorm_rope");
  return {q, k, v};
}

// triton_npu/torch_api/npu_triton_causal_conv1d_update.cpp:22-138.  As there
// (`(void)activation`, :38: the kernel is built with SiLU), SiLU is always
// applied; the C-ABI xk_causal_conv1d_update keeps an activation switch.
torch::Tensor npu_causal_conv1d_update(
    torch::Tensor& x, torch::Tensor& conv_state, torch::Tensor& weight, bool /*activation*/,
    const std::optional<torch::Tensor>& bias, const std::optional<torch::Tensor>& cache_seqlens,
    const std::optional<torch::Tensor>& conv_state_indices,
    const std::optional<torch::Tensor>& num_accepted_tokens,
    const std::optional<torch::Tensor>& query_start_loc, int32_t /*max_query_len*/,
    const std::optional<torch::Tensor>& /*intermediate_conv_window*/, int32_t pad_slot_id,
    bool /*validate_data*/) {
  if (has(query_start_loc)) {  // reference :41-45
    TORCH_WARN("npu_causal_conv1d_update does not support query_start_loc");
    return torch::zeros({1});
  }
  TORCH_CHECK(!has(cache_seqlens) && !has(num_accepted_tokens),
              "causal_conv1d_update does not support cache_seqlens or num_accepted_tokens");
  const bool unsq = x.dim() == 2;
  auto xs = unsq ? x.unsqueeze(-1) : x;
  TORCH_CHECK(xs.dim() == 3, "causal_conv1d_update expects x [B, D] or [B, D, T]");
  const int64_t B = xs.size(0), D = xs.size(1), T = xs.size(2);
  const int64_t W = weight.size(1), S = conv_state.size(2);
  TORCH_CHECK(weight.size(0) == D && conv_state.size(1) == D, "weight / conv_state dim mismatch");
  auto out = torch::empty_like(xs);
  torch::Tensor idx;
  if (has(conv_state_indices)) idx = conv_state_indices->to(torch::kInt32).contiguous();
  auto w = (weight.scalar_type() == x.scalar_type() || weight.scalar_type() == torch::kFloat32)
               ? weight
               : weight.to(x.scalar_type());
  torch::Tensor b;
  if (has(bias)) b = bias->to(w.scalar_type()).contiguous();
  check(xk_causal_conv1d_update(xs.data_ptr(), xs.stride(0), xs.stride(1), xs.stride(2),
                                conv_state.data_ptr(), conv_state.stride(0), conv_state.stride(1),
                                conv_state.stride(2), w.data_ptr(), w.stride(0), w.stride(1),
                                ptr(b), xdt(w), static_cast<const int32_t*>(ptr(idx)),
                                pad_slot_id, conv_state.size(0), out.data_ptr(), out.stride(0),
                                out.stride(1), out.stride(2), B, D, T, W, S, /*activation=*/1,
                                xdt(xs),
                                stream_of(x)),
        "xk_causal_conv1d_update");
  return unsq ? out.squeeze(-1) : out;
}

// triton_npu/torch_api/npu_triton_causal_conv1d_update_v2.cpp:99-239
torch::Tensor npu_causal_conv1d_update_v2(
    torch::Tensor& x, torch::Tensor& conv_state, torch::Tensor& weight, bool activation,
    const std::optional<torch::Tensor>& bias,
    const std::optional<torch::Tensor>& conv_state_indices,
    const std::optional<torch::Tensor>& query_start_loc, int32_t max_query_len,
    int32_t pad_slot_id, const std::optional<torch::Tensor>& block_idx_last_scheduled_token,
    const std::optional<torch::Tensor>& initial_state_idx, bool /*validate_data*/,
    const std::optional<torch::Tensor>& num_accepted_tokens) {
  TORCH_CHECK(weight.dim() == 2, "causal_conv1d_update_v2 expects weight shape [dim, width].");
  TORCH_CHECK(has(block_idx_last_scheduled_token) == has(initial_state_idx),
              "causal_conv1d_update_v2 expects both APC tensors or neither.");
  TORCH_CHECK(conv_state.dim() == 3,
              "causal_conv1d_update_v2 expects conv_state shape [num_cache_lines, dim, state_len].");
  const bool dense = !has(query_start_loc);
  bool unsq = false;
  int64_t B, D, T = 0, mql;
  torch::Tensor xt, qsl;
  if (dense) {
    unsq = x.dim() == 2;
    auto xw = unsq ? x.unsqueeze(-1) : x;
    B = xw.size(0);
    D = xw.size(1);
    T = xw.size(2);
    xt = xw.transpose(1, 2).contiguous().view({B * T, D});
    qsl = torch::arange(0, (B + 1) * T, T, x.options().dtype(torch::kInt32));
    mql = T;
  } else {
    TORCH_CHECK(x.dim() == 2, "causal_conv1d_update_v2 expects x to be 2D [num_tokens, dim] "
                              "when query_start_loc is provided.");
    qsl = query_start_loc->to(torch::kInt32).contiguous();
    B = qsl.numel() - 1;
    D = x.size(1);
    xt = x.stride(1) == 1 ? x : x.contiguous();
    mql = max_query_len;
    if (mql < 0)
      mql = B > 0 ? (qsl.slice(0, 1) - qsl.slice(0, 0, -1)).max().item<int64_t>() : 0;
  }
  const int64_t W = weight.size(1);
  TORCH_CHECK(W >= 1 && W <= 6, "causal_conv1d_update_v2 expects width in [1, 6], got ", W);
  TORCH_CHECK(weight.size(0) == D && conv_state.size(1) == D, "weight / conv_state dim mismatch");
  torch::Tensor slots;
  int64_t sstride = 0;
  int s2d = 0;
  if (has(conv_state_indices)) {
    slots = conv_state_indices->to(torch::kInt32).contiguous();
    s2d = slots.dim() == 2;
    sstride = s2d ? slots.stride(0) : 1;
    TORCH_CHECK(slots.size(0) == B, "conv_state_indices batch mismatch");
  }
  torch::Tensor last, init, acc;
  if (has(block_idx_last_scheduled_token)) {
    last = block_idx_last_scheduled_token->to(torch::kInt32).contiguous();
    init = initial_state_idx->to(torch::kInt32).contiguous();
  }
  if (has(num_accepted_tokens)) acc = num_accepted_tokens->to(torch::kInt32).contiguous();
  // x is read in the state's dtype (reference :172), the result returned in
  // x's own dtype (:238).
  const auto x_dtype = x.scalar_type();
  if (xt.scalar_type() != conv_state.scalar_type()) xt = xt.to(conv_state.scalar_type());
  auto w = (weight.scalar_type() == xt.scalar_type() || weight.scalar_type() == torch::kFloat32)
               ? weight
               : weight.to(xt.scalar_type());
  torch::Tensor b;
  if (has(bias)) b = bias->to(w.scalar_type()).contiguous();
  auto out = torch::empty_like(xt);
  check(xk_causal_conv1d_varlen(
            xt.data_ptr(), xt.stride(0), xt.size(0), out.data_ptr(), out.stride(0),
            conv_state.data_ptr(), conv_state.stride(0), conv_state.stride(1),
            conv_state.stride(2), conv_state.size(0), conv_state.size(2), w.data_ptr(),
            w.stride(0), w.stride(1), ptr(b), xdt(w),
            static_cast<const int32_t*>(qsl.data_ptr()), B,
            static_cast<const int32_t*>(ptr(slots)), sstride, s2d,
            static_cast<const int32_t*>(ptr(init)), static_cast<const int32_t*>(ptr(last)),
            static_cast<const int32_t*>(ptr(acc)), D, W, mql, 0, activation, pad_slot_id,
            xdt(xt), stream_of(x)),
        "xk_causal_conv1d_varlen");
  out = out.to(x_dtype);
  if (dense) {
    auto o = out.view({B, T, D}).transpose(1, 2);
    return unsq ? o.squeeze(-1) : o.contiguous();
  }
  return out;
}

// triton_npu/torch_api/npu_triton_recurrent_gated_delta_rule.cpp:54-247.
// use_qk_l2norm_in_kernel is accepted and ignored, as there: the reference
// never passes it to its kernel, which is built with the normalisation on
// (:216-238; test_fused_recurrent_gated_delta_rule.py:731), so q and k are
// always l2-normalised.  The C-ABI xk_gdn_recurrent keeps the switch.
std::pair<torch::Tensor, torch::Tensor> npu_fused_recurrent_gated_delta_rule(
    torch::Tensor& q, torch::Tensor& k, torch::Tensor& v, torch::Tensor& g,
    const std::optional<torch::Tensor>& beta, const std::optional<float>& scale,
    const std::optional<torch::Tensor>& initial_state, bool inplace_final_state,
    const std::optional<torch::Tensor>& cu_seqlens,
    const std::optional<torch::Tensor>& ssm_state_indices,
    const std::optional<torch::Tensor>& num_accepted_tokens, bool /*use_qk_l2norm_in_kernel*/) {
  const int64_t B = k.size(0), T = k.size(1), H = k.size(2), K = k.size(3);
  const int64_t HV = v.size(2), V = v.size(3);
  TORCH_CHECK(has(cu_seqlens) || q.size(0) == 1,
              "batch size is not 1 when cu_seqlens is not provided");
  TORCH_CHECK(has(initial_state), "initial_state must be provided");
  const float sc = scale.has_value() ? *scale : 1.0f / std::sqrt(static_cast<float>(K));
  const int64_t N = has(cu_seqlens) ? cu_seqlens->numel() - 1 : B;
  auto qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous(), gc = g.contiguous();
  torch::Tensor bc;
  if (has(beta)) bc = beta->contiguous();
  auto o = torch::empty({B, T, HV, V}, q.options());
  const torch::Tensor& h0 = *initial_state;
  TORCH_CHECK(h0.scalar_type() == torch::kFloat32 && h0.is_contiguous(),
              "initial_state must be contiguous float32");
  torch::Tensor fin = inplace_final_state
                          ? h0
                          : torch::empty({N, HV, K, V}, q.options().dtype(torch::kFloat32));
  torch::Tensor idx, acc, cu;
  int64_t s0 = 0, s1 = 0;
  if (has(ssm_state_indices)) {
    idx = ssm_state_indices->to(torch::kInt32).contiguous();
    s0 = idx.stride(0);
    s1 = idx.dim() == 2 ? idx.stride(1) : 0;
  }
  if (has(num_accepted_tokens)) acc = num_accepted_tokens->to(torch::kInt32).contiguous();
  if (has(cu_seqlens)) cu = cu_seqlens->contiguous();
  check(xk_gdn_recurrent(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), xdt(qc), gc.data_ptr(),
                         xdt(gc), ptr(bc), bc.defined() ? xdt(bc) : XK_F32, o.data_ptr(),
                         static_cast<const float*>(h0.data_ptr()), h0.stride(0),
                         static_cast<float*>(fin.data_ptr()), fin.stride(0), h0.size(0), ptr(cu),
                         cu.defined() ? xdt(cu) : XK_I32,
                         static_cast<const int32_t*>(ptr(idx)), s0, s1,
                         static_cast<const int32_t*>(ptr(acc)), N, cu.defined() ? 0 : T, H, HV,
                         K, V, sc, /*use_qk_l2norm=*/1, inplace_final_state, stream_of(q)),
        "xk_gdn_recurrent");
  return {o, fin};
}

// triton_npu/torch_api/npu_triton_rope_inplace.cpp:22-64
void rope_inplace(torch::Tensor& x, torch::Tensor& sin, torch::Tensor& cos, uint32_t rope_dim) {
  auto org_shape = x.sizes().vec();
  int64_t bsz = 0, head_num = 0, hidden_size = 0;
  if (x.dim() == 2) {
    bsz = x.size(0);
    head_num = 1;
    hidden_size = x.size(1);
  } else if (x.dim() == 3) {
    bsz = x.size(0);
    head_num = x.size(1);
    hidden_size = x.size(2);
    x = x.view({-1, hidden_size});
  }
  TORCH_CHECK(bsz > 0 || x.numel() == 0, "rope_inplace expects a 2-D or 3-D x");
  TORCH_CHECK(x.stride(-1) == 1, "rope_inplace needs rows with unit column stride");
  TORCH_CHECK(sin.stride(-1) == 1 && cos.stride(-1) == 1 && sin.stride(0) == cos.stride(0),
              "sin and cos must share a row stride with unit column stride");
  check(xk_rope_inplace(x.data_ptr(), bsz * head_num, head_num, x.stride(0), hidden_size,
                        sin.data_ptr(), cos.data_ptr(), cos.stride(0), rope_dim, xdt(x),
                        xdt(sin), stream_of(x)),
        "xk_rope_inplace");
  if (org_shape.size() == 3) x = x.view(org_shape);
}

// triton_npu/torch_api/npu_triton_fused_gdn_gating.cpp:33-94
std::pair<torch::Tensor, torch::Tensor> npu_fused_gdn_gating(torch::Tensor& A_log,
                                                             torch::Tensor& a, torch::Tensor& b,
                                                             torch::Tensor& dt_bias, float beta,
                                                             float threshold) {
  for (auto [t, name] : {std::pair<const torch::Tensor*, const char*>{&A_log, "A_log"},
                         {&a, "a"}, {&b, "b"}, {&dt_bias, "dt_bias"}}) {
    TORCH_CHECK(t->defined(), name, " tensor is not defined");
    TORCH_CHECK(t->is_contiguous(), name, " tensor must be contiguous");
  }
  TORCH_CHECK(A_log.scalar_type() == torch::kFloat32, "A_log must be float32");
  TORCH_CHECK(dt_bias.scalar_type() == torch::kFloat32, "dt_bias must be float32");
  TORCH_CHECK(A_log.dim() == 1, "A_log must be 1D tensor");
  TORCH_CHECK(a.dim() == 2, "a must be 2D tensor (batch, num_heads)");
  TORCH_CHECK(b.dim() == 2, "b must be 2D tensor (batch, num_heads)");
  TORCH_CHECK(dt_bias.dim() == 1, "dt_bias must be 1D tensor");
  TORCH_CHECK(a.sizes() == b.sizes() && a.scalar_type() == b.scalar_type(),
              "a and b must have the same shape and dtype");
  const int64_t batch = a.size(0), num_heads = a.size(1);
  auto g = torch::empty({1, batch, num_heads}, a.options().dtype(torch::kFloat32));
  auto beta_output = torch::empty({1, batch, num_heads}, b.options());
  check(xk_fused_gdn_gating(static_cast<const float*>(A_log.data_ptr()), a.data_ptr(),
                            b.data_ptr(), static_cast<const float*>(dt_bias.data_ptr()),
                            static_cast<float*>(g.data_ptr()), beta_output.data_ptr(), batch,
                            num_heads, beta, threshold, xdt(a), stream_of(a)),
        "xk_fused_gdn_gating");
  return {g, beta_output};
}

// triton_npu/torch_api/npu_triton_fused_sigmoid_gating_delta_rule_update.cpp:54-177.
// use_qk_l2norm_in_kernel is accepted and ignored, as there: the wrapper
// never passes it to its kernel (:141-165), whose binary is built by the
// test that calls it with True (test_fused_sigmoid_gating_delta_rule_update.py:
// 268-295), so q and k are always l2-normalised.  The C-ABI keeps the switch.
torch::Tensor npu_fused_sigmoid_gating_delta_rule_update(
    torch::Tensor& A_log, torch::Tensor& a, torch::Tensor& dt_bias, torch::Tensor& q,
    torch::Tensor& k, torch::Tensor& v, torch::Tensor& b, torch::Tensor& initial_state_source,
    torch::Tensor& initial_state_indices, torch::Tensor& cu_seqlens,
    const std::optional<float>& scale, bool /*use_qk_l2norm_in_kernel*/, float softplus_beta,
    float softplus_threshold) {
  for (auto [t, name] : {std::pair<const torch::Tensor*, const char*>{&A_log, "A_log"},
                         {&a, "a"}, {&dt_bias, "dt_bias"}, {&q, "q"}, {&k, "k"}, {&v, "v"},
                         {&b, "b"}, {&initial_state_source, "initial_state_source"},
                         {&initial_state_indices, "initial_state_indices"},
                         {&cu_seqlens, "cu_seqlens"}}) {
    TORCH_CHECK(t->defined(), name, " must be defined");
    TORCH_CHECK(t->is_contiguous(), name, " must be contiguous");
  }
  TORCH_CHECK(q.dim() == 4, "q must be 4D [B, T, H, K]");
  TORCH_CHECK(k.dim() == 4, "k must be 4D [B, T, H, K]");
  TORCH_CHECK(v.dim() == 4, "v must be 4D [B, T, HV, V]");
  TORCH_CHECK(a.dim() == 3, "a must be 3D [B, T, HV]");
  TORCH_CHECK(b.dim() == 3, "b must be 3D [B, T, HV]");
  TORCH_CHECK(A_log.dim() == 1, "A_log must be 1D [HV]");
  TORCH_CHECK(dt_bias.dim() == 1, "dt_bias must be 1D [HV]");
  TORCH_CHECK(initial_state_source.dim() == 4,
              "initial_state_source must be 4D [slots, HV, K, V]");
  TORCH_CHECK(initial_state_indices.dim() == 1, "initial_state_indices must be 1D [N]");
  TORCH_CHECK(cu_seqlens.dim() == 1, "cu_seqlens must be 1D [N + 1]");
  const int64_t B = k.size(0), T = k.size(1), H = k.size(2), K = k.size(3);
  const int64_t HV = v.size(2), V = v.size(3);
  const int64_t N = cu_seqlens.numel() - 1;
  TORCH_CHECK(q.sizes() == k.sizes(), "q/k shape mismatch");
  TORCH_CHECK(v.size(0) == B && v.size(1) == T, "v B/T mismatch");
  TORCH_CHECK(a.size(0) == B && a.size(1) == T && a.size(2) == HV, "a shape mismatch");
  TORCH_CHECK(b.sizes() == a.sizes(), "a/b shape mismatch");
  TORCH_CHECK(A_log.numel() == HV, "A_log HV mismatch");
  TORCH_CHECK(dt_bias.numel() == HV, "dt_bias HV mismatch");
  TORCH_CHECK(initial_state_source.size(1) == HV && initial_state_source.size(2) == K &&
                  initial_state_source.size(3) == V,
              "initial_state_source shape mismatch");
  TORCH_CHECK(initial_state_indices.numel() == N,
              "initial_state_indices size must equal cu_seqlens size - 1");
  TORCH_CHECK(HV % H == 0, "HV must be divisible by H");
  TORCH_CHECK(A_log.scalar_type() == torch::kFloat32, "A_log must be float32");
  TORCH_CHECK(dt_bias.scalar_type() == torch::kFloat32, "dt_bias must be float32");
  TORCH_CHECK(initial_state_source.scalar_type() == torch::kFloat32,
              "initial_state_source must be float32");
  TORCH_CHECK(initial_state_indices.scalar_type() == torch::kInt32,
              "initial_state_indices must be int32");
  TORCH_CHECK(cu_seqlens.scalar_type() == torch::kInt32, "cu_seqlens must be int32");
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "a and b must have the same dtype");
  const float sc = scale.has_value() ? *scale : 1.0f / std::sqrt(static_cast<float>(K));
  auto o = torch::empty({B, T, HV, V}, q.options());
  check(xk_gdn_sigmoid_gating_update(
            static_cast<const float*>(A_log.data_ptr()), a.data_ptr(),
            static_cast<const float*>(dt_bias.data_ptr()), softplus_beta, softplus_threshold,
            q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(), xdt(a), o.data_ptr(),
            static_cast<float*>(initial_state_source.data_ptr()), initial_state_source.stride(0),
            initial_state_source.size(0),
            static_cast<const int32_t*>(initial_state_indices.data_ptr()),
            static_cast<const int32_t*>(cu_seqlens.data_ptr()), N, H, HV, K, V, sc,
            /*use_qk_l2norm=*/1, xdt(q), stream_of(q)),
        "xk_gdn_sigmoid_gating_update");
  return o;
}

// triton_npu/torch_api/npu_triton_fused_qkvzba_split_reshape.cpp:116-230
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor>
npu_fused_qkvzba_split_reshape_cat(torch::Tensor& mixed_qkvz, torch::Tensor& mixed_ba,
                                   int32_t num_heads_qk, int32_t num_heads_v, int32_t head_qk,
                                   int32_t head_v) {
  const int64_t rows = mixed_qkvz.size(0);
  const int32_t v_heads_per_qk = num_heads_v / num_heads_qk;
  TORCH_CHECK(v_heads_per_qk >= 1 && v_heads_per_qk <= 4 && num_heads_v % num_heads_qk == 0,
              "npu_fused_qkvzba_split_reshape_cat only supports v_heads_per_qk in [1, 4], "
              "but got ", v_heads_per_qk, " for num_heads_qk=", num_heads_qk,
              " num_heads_v=", num_heads_v);
  auto q2 = rows_of(mixed_qkvz, rows);
  auto b2 = rows_of(mixed_ba, rows);
  const int64_t qkv_dim = static_cast<int64_t>(num_heads_qk) * head_qk * 2 +
                          static_cast<int64_t>(num_heads_v) * head_v;
  auto mixed_qkv = torch::empty({rows, qkv_dim}, mixed_qkvz.options());
  auto z_flat = torch::empty({rows, static_cast<int64_t>(num_heads_v) * head_v},
                             mixed_qkvz.options());
  auto b = torch::empty({rows, num_heads_v}, mixed_ba.options());
  auto a = torch::empty({rows, num_heads_v}, mixed_ba.options());
  check(xk_fused_qkvzba_split_reshape_cat(q2.data_ptr(), q2.stride(0), b2.data_ptr(),
                                          b2.stride(0), mixed_qkv.data_ptr(), z_flat.data_ptr(),
                                          b.data_ptr(), a.data_ptr(), rows, num_heads_qk,
                                          num_heads_v, head_qk, head_v, xdt(q2), xdt(b2),
                                          stream_of(mixed_qkvz)),
        "xk_fused_qkvzba_split_reshape_cat");
  auto z = z_flat.view({rows, num_heads_v, head_v});
  return {mixed_qkv, z, b, a};
}

// triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:556-642
std::pair<torch::Tensor, torch::Tensor> npu_chunk_gated_delta_rule(
    torch::Tensor& q, torch::Tensor& k, torch::Tensor& v, torch::Tensor& g, torch::Tensor& beta,
    const std::optional<float>& scale, const std::optional<torch::Tensor>& initial_state,
    bool output_final_state, const std::optional<torch::Tensor>& cu_seqlens, bool head_first,
    bool use_qk_l2norm_in_kernel) {
  TORCH_CHECK(!head_first, "chunk_gated_delta_rule torch_api only supports head_first=false.");
  TORCH_CHECK(q.scalar_type() == torch::kBFloat16 && k.scalar_type() == torch::kBFloat16 &&
                  v.scalar_type() == torch::kBFloat16,
              "chunk_gated_delta_rule expects q/k/v to be bfloat16.");
  if (has(initial_state)) {  // reference :574-579
    const auto st = initial_state->scalar_type();
    TORCH_CHECK(st == torch::kBFloat16 || st == torch::kFloat32,
                "chunk_gated_delta_rule expects initial_state to be bfloat16 or float32, got ",
                st);
  }
  const int64_t B = q.size(0), T = q.size(1), H = q.size(2), K = q.size(3);
  const int64_t HV = v.size(2), V = v.size(3);
  TORCH_CHECK(q.sizes() == k.sizes(), "q and k must have the same shape.");
  TORCH_CHECK(HV % H == 0, "chunk_gated_delta_rule expects num_heads_v to be divisible by "
                           "num_heads_qk, got ", HV, " and ", H);
  TORCH_CHECK(beta.dim() == 3 && beta.size(0) == B && beta.size(1) == T && beta.size(2) == HV,
              "beta must have shape [B, T, H].");
  TORCH_CHECK(g.dim() == 3 && g.size(0) == B && g.size(1) == T && g.size(2) == HV,
              "g must have shape [B, T, H].");
  auto [cu, N] = seqs(B, T, cu_seqlens, q.device());
  const float sc = scale.has_value() ? *scale : std::pow(static_cast<float>(K), -0.5f);
  auto qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous();
  auto gc = g.contiguous(), bc = beta.contiguous();
  torch::Tensor h0;
  if (has(initial_state)) h0 = initial_state->to(torch::kFloat32).contiguous();
  auto f32 = q.options().dtype(torch::kFloat32);
  torch::Tensor fin = output_final_state ? torch::empty({N, HV, K, V}, f32) : torch::Tensor();
  auto o = torch::empty({B, T, HV, V}, q.options());
  auto ws = workspace(xk_gdn_chunk_workspace_bytes(B * T, N, HV), q.device());
  check(xk_gdn_chunk_fwd(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), xdt(qc), gc.data_ptr(),
                         xdt(gc), bc.data_ptr(), xdt(bc), o.data_ptr(),
                         static_cast<const float*>(ptr(h0)), static_cast<float*>(mptr(fin)),
                         cu.data_ptr(), xdt(cu), N, B * T, H, HV, K, V, sc,
                         use_qk_l2norm_in_kernel, ws.data_ptr(), ws.numel(), stream_of(q)),
        "xk_gdn_chunk_fwd");
  return {o, fin};
}

// triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:151-227
torch::Tensor npu_chunk_local_cumsum(const torch::Tensor& g, int64_t chunk_size,
                                     const std::optional<torch::Tensor>& cu_seqlens) {
  TORCH_CHECK(g.dim() == 3, "chunk_local_cumsum expects g to have shape [B, T, H].");
  TORCH_CHECK(chunk_size > 0 && (chunk_size & (chunk_size - 1)) == 0,
              "chunk_local_cumsum expects chunk_size to be a power of two, got ", chunk_size);
  const int64_t B = g.size(0), T = g.size(1), H = g.size(2);
  auto [cu, N] = seqs(B, T, cu_seqlens, g.device());
  auto gc = g.contiguous();
  auto out = torch::empty(g.sizes(), g.options().dtype(torch::kFloat32));
  check(xk_chunk_local_cumsum(gc.data_ptr(), xdt(gc), static_cast<float*>(out.data_ptr()),
                              B * T, H, cu.data_ptr(), xdt(cu), N, chunk_size, stream_of(g)),
        "xk_chunk_local_cumsum");
  return out;
}

// triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:229-297
torch::Tensor npu_chunk_scaled_dot_kkt_fwd(const torch::Tensor& k, const torch::Tensor& beta,
                                           const torch::Tensor& g_cumsum, int64_t chunk_size,
                                           const std::optional<torch::Tensor>& cu_seqlens) {
  TORCH_CHECK(chunk_size == 64, "chunk_scaled_dot_kkt_fwd supports chunk_size=64");
  const int64_t B = k.size(0), T = k.size(1), Hg = k.size(2), K = k.size(3), H = beta.size(2);
  auto [cu, N] = seqs(B, T, cu_seqlens, k.device());
  auto kc = k.contiguous(), bc = beta.contiguous();
  torch::Tensor gc;
  if (g_cumsum.defined()) gc = g_cumsum.to(torch::kFloat32).contiguous();
  auto A = torch::empty({B, T, H, 64}, k.options().dtype(torch::kFloat32));
  auto ws = workspace(xk_gdn_stage_workspace_bytes(N), k.device());
  check(xk_chunk_scaled_dot_kkt(kc.data_ptr(), xdt(kc), bc.data_ptr(), xdt(bc),
                                static_cast<const float*>(ptr(gc)),
                                static_cast<float*>(A.data_ptr()), B * T, Hg, H, K,
                                cu.data_ptr(), xdt(cu), N, ws.data_ptr(), ws.numel(),
                                stream_of(k)),
        "xk_chunk_scaled_dot_kkt");
  return A;
}

// triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:299-395
torch::Tensor npu_solve_tril(const torch::Tensor& A, int64_t chunk_size,
                             const std::optional<torch::Tensor>& cu_seqlens,
                             torch::ScalarType output_dtype) {
  TORCH_CHECK(chunk_size == 64,
              "chunk_gated_delta_rule solve_tril wrapper only supports chunk_size=64.");
  TORCH_CHECK(A.dim() == 4 && A.size(3) == 64, "solve_tril expects A of shape [B, T, H, 64]");
  const int64_t B = A.size(0), T = A.size(1), H = A.size(2);
  auto [cu, N] = seqs(B, T, cu_seqlens, A.device());
  auto Ac = A.to(torch::kFloat32).contiguous();
  auto Ai = torch::empty(A.sizes(), A.options().dtype(output_dtype));
  auto ws = workspace(xk_gdn_stage_workspace_bytes(N), A.device());
  check(xk_solve_tril(static_cast<const float*>(Ac.data_ptr()), Ai.data_ptr(), xdt(Ai), B * T, H,
                      cu.data_ptr(), xdt(cu), N, ws.data_ptr(), ws.numel(), stream_of(A)),
        "xk_solve_tril");
  return Ai;
}

// triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:397-475
std::pair<torch::Tensor, torch::Tensor> npu_recompute_w_u_fwd(
    const torch::Tensor& k, const torch::Tensor& v, const torch::Tensor& beta,
    const torch::Tensor& g_cumsum, const torch::Tensor& A,
    const std::optional<torch::Tensor>& cu_seqlens) {
  const int64_t B = k.size(0), T = k.size(1), Hg = k.size(2), K = k.size(3);
  const int64_t H = v.size(2), V = v.size(3);
  auto [cu, N] = seqs(B, T, cu_seqlens, k.device());
  auto kc = k.contiguous(), vc = v.contiguous(), bc = beta.contiguous(), Ac = A.contiguous();
  auto gc = g_cumsum.to(torch::kFloat32).contiguous();
  auto w = torch::empty({B, T, H, K}, k.options());
  auto u = torch::empty_like(vc);
  auto ws = workspace(xk_gdn_stage_workspace_bytes(N), k.device());
  check(xk_recompute_w_u(kc.data_ptr(), vc.data_ptr(), xdt(kc), bc.data_ptr(), xdt(bc),
                         static_cast<const float*>(gc.data_ptr()), Ac.data_ptr(), xdt(Ac),
                         w.data_ptr(), u.data_ptr(), B * T, Hg, H, K, V, cu.data_ptr(), xdt(cu),
                         N, ws.data_ptr(), ws.numel(), stream_of(k)),
        "xk_recompute_w_u");
  return {w, u};
}

// triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:644-802
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> npu_chunk_gated_delta_rule_fwd_h(
    torch::Tensor& k, torch::Tensor& w, torch::Tensor& u, const std::optional<torch::Tensor>& g,
    const std::optional<torch::Tensor>& initial_state, bool output_final_state,
    int64_t chunk_size, bool save_new_value, const std::optional<torch::Tensor>& cu_seqlens,
    const std::optional<torch::Tensor>& chunk_offsets) {
  TORCH_CHECK(chunk_size == 64, "chunk_gated_delta_rule_fwd_h only supports chunk_size=64");
  TORCH_CHECK(k.scalar_type() == torch::kBFloat16,
              "chunk_gated_delta_rule_fwd_h expects k to be bfloat16, got ", k.scalar_type());
  TORCH_CHECK(w.scalar_type() == torch::kBFloat16,
              "chunk_gated_delta_rule_fwd_h expects w to be bfloat16, got ", w.scalar_type());
  TORCH_CHECK(u.scalar_type() == torch::kBFloat16,
              "chunk_gated_delta_rule_fwd_h expects u to be bfloat16, got ", u.scalar_type());
  const int64_t B = k.size(0), T = k.size(1), Hg = k.size(2), K = k.size(3);
  const int64_t H = u.size(2), V = u.size(3);
  auto [cu, N] = seqs(B, T, cu_seqlens, k.device());
  TORCH_CHECK(!has(chunk_offsets) || chunk_offsets->numel() == N + 1,
              "chunk_offsets must have N + 1 entries");
  const int64_t NT = num_chunks(cu, B * T);
  auto kc = k.contiguous(), wc = w.contiguous(), uc = u.contiguous();
  torch::Tensor gc, h0;
  if (has(g)) gc = g->to(torch::kFloat32).contiguous();
  if (has(initial_state)) h0 = initial_state->to(torch::kFloat32).contiguous();
  const int64_t hb = has(cu_seqlens) ? 1 : B;
  auto h = torch::empty({hb, NT / hb, H, K, V}, k.options());
  torch::Tensor v_new = save_new_value ? torch::empty_like(uc) : torch::Tensor();
  torch::Tensor fin = output_final_state
                          ? torch::empty({N, H, K, V}, k.options().dtype(torch::kFloat32))
                          : torch::Tensor();
  auto ws = workspace(xk_gdn_stage_workspace_bytes(N), k.device());
  check(xk_chunk_fwd_h(kc.data_ptr(), wc.data_ptr(), uc.data_ptr(), xdt(kc),
                       static_cast<const float*>(ptr(gc)), static_cast<const float*>(ptr(h0)),
                       h.data_ptr(), NT, mptr(v_new), static_cast<float*>(mptr(fin)), B * T, Hg,
                       H, K, V, cu.data_ptr(), xdt(cu), N, ws.data_ptr(), ws.numel(),
                       stream_of(k)),
        "xk_chunk_fwd_h");
  return {h, v_new, fin};
}

// triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:477-554
torch::Tensor npu_chunk_fwd_o(const torch::Tensor& q, const torch::Tensor& k,
                              const torch::Tensor& v, const torch::Tensor& h,
                              const torch::Tensor& g_cumsum, float scale, int64_t chunk_size,
                              const std::optional<torch::Tensor>& cu_seqlens) {
  TORCH_CHECK(chunk_size == 64, "chunk_fwd_o supports chunk_size=64");
  const int64_t B = q.size(0), T = q.size(1), Hg = q.size(2), K = q.size(3);
  const int64_t H = v.size(2), V = v.size(3);
  auto [cu, N] = seqs(B, T, cu_seqlens, q.device());
  auto qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous(), hc = h.contiguous();
  const int64_t NT = hc.numel() / (H * K * V);
  torch::Tensor gc;
  if (g_cumsum.defined()) gc = g_cumsum.to(torch::kFloat32).contiguous();
  auto o = torch::empty_like(vc);
  auto ws = workspace(xk_gdn_stage_workspace_bytes(N), q.device());
  check(xk_chunk_fwd_o(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), hc.data_ptr(), NT, xdt(qc),
                       static_cast<const float*>(ptr(gc)), o.data_ptr(), scale, B * T, Hg, H, K,
                       V, cu.data_ptr(), xdt(cu), N, ws.data_ptr(), ws.numel(), stream_of(q)),
        "xk_chunk_fwd_o");
  return o;
}

namespace {

// Checks shared by the two fused decode steps: the kernels index ssm_state
// as dense fp32 [slots, HV, K, V] (slot stride from stride(0)) and
// conv_state in mixed_qkv's dtype.
void check_conv_decode(const torch::Tensor& mixed_qkv, const torch::Tensor& conv_state,
                       const torch::Tensor& conv_weight, const torch::Tensor& ssm_state,
                       int64_t num_heads_qk, int64_t num_heads_v, int64_t head_k,
                       int64_t head_v) {
  TORCH_CHECK(mixed_qkv.dim() == 2, "gdn_conv_decode expects mixed_qkv [B, D]");
  const int64_t D = mixed_qkv.size(1);
  TORCH_CHECK(D == 2 * num_heads_qk * head_k + num_heads_v * head_v,
              "mixed_qkv width does not match the head layout");
  TORCH_CHECK(ssm_state.scalar_type() == torch::kFloat32, "ssm_state must be float32");
  TORCH_CHECK(ssm_state.dim() == 4 && ssm_state.size(1) == num_heads_v &&
                  ssm_state.size(2) == head_k && ssm_state.size(3) == head_v,
              "ssm_state must have shape [slots, num_heads_v, head_k, head_v]");
  TORCH_CHECK(ssm_state.stride(3) == 1 && ssm_state.stride(2) == head_v &&
                  ssm_state.stride(1) == head_k * head_v,
              "ssm_state must be contiguous within each slot");
  TORCH_CHECK(conv_state.scalar_type() == mixed_qkv.scalar_type(),
              "conv_state must have mixed_qkv's dtype");
  TORCH_CHECK(conv_state.dim() == 3 && conv_state.size(1) == D,
              "conv_state must have shape [lines, D, state_len]");
  TORCH_CHECK(conv_weight.dim() == 2 && conv_weight.size(0) == D,
              "conv_weight must have shape [D, width]");
}

}  // namespace

torch::Tensor npu_gdn_conv_decode(
    torch::Tensor& mixed_qkv, torch::Tensor& conv_state, torch::Tensor& conv_weight,
    torch::Tensor& g, const std::optional<torch::Tensor>& beta, torch::Tensor& ssm_state,
    int64_t num_heads_qk, int64_t num_heads_v, int64_t head_k, int64_t head_v,
    const std::optional<float>& scale, const std::optional<torch::Tensor>& conv_bias,
    const std::optional<torch::Tensor>& conv_state_indices,
    const std::optional<torch::Tensor>& ssm_state_indices, int32_t pad_slot_id,
    bool use_qk_l2norm) {
  check_conv_decode(mixed_qkv, conv_state, conv_weight, ssm_state, num_heads_qk, num_heads_v,
                    head_k, head_v);
  const int64_t B = mixed_qkv.size(0);
  TORCH_CHECK(g.dim() == 2 && g.size(0) == B && g.size(1) == num_heads_v,
              "g must have shape [B, num_heads_v]");
  TORCH_CHECK(!has(beta) || (beta->dim() == 2 && beta->size(0) == B &&
                             beta->size(1) == num_heads_v),
              "beta must have shape [B, num_heads_v]");
  const float sc = scale.has_value() ? *scale : 1.0f / std::sqrt(static_cast<float>(head_k));
  auto x = mixed_qkv.stride(1) == 1 ? mixed_qkv : mixed_qkv.contiguous();
  torch::Tensor cb, ci, si, bc;
  if (has(conv_bias)) cb = conv_bias->to(conv_weight.scalar_type()).contiguous();
  if (has(conv_state_indices)) ci = conv_state_indices->to(torch::kInt32).contiguous();
  if (has(ssm_state_indices)) si = ssm_state_indices->to(torch::kInt32).contiguous();
  if (has(beta)) bc = beta->contiguous();
  auto gc = g.contiguous();
  auto o = torch::empty({B, num_heads_v, head_v}, x.options());
  check(xk_gdn_conv_decode(x.data_ptr(), x.stride(0), conv_state.data_ptr(), conv_state.stride(0),
                           conv_state.stride(1), conv_state.stride(2), conv_state.size(0),
                           conv_state.size(2), conv_weight.data_ptr(), conv_weight.stride(0),
                           conv_weight.stride(1), ptr(cb), xdt(conv_weight), conv_weight.size(1),
                           static_cast<const int32_t*>(ptr(ci)), pad_slot_id, gc.data_ptr(),
                           xdt(gc), ptr(bc), bc.defined() ? xdt(bc) : XK_F32,
                           static_cast<float*>(ssm_state.data_ptr()), ssm_state.stride(0),
                           ssm_state.size(0), static_cast<const int32_t*>(ptr(si)),
                           o.data_ptr(), B, num_heads_qk, num_heads_v, head_k, head_v, sc,
                           use_qk_l2norm, xdt(x), stream_of(x)),
        "xk_gdn_conv_decode");
  return o;
}

torch::Tensor npu_gdn_conv_sigmoid_gating_decode(
    torch::Tensor& mixed_qkv, torch::Tensor& conv_state, torch::Tensor& conv_weight,
    torch::Tensor& A_log, torch::Tensor& a, torch::Tensor& dt_bias, torch::Tensor& b,
    torch::Tensor& ssm_state, int64_t num_heads_qk, int64_t num_heads_v, int64_t head_k,
    int64_t head_v, const std::optional<float>& scale,
    const std::optional<torch::Tensor>& conv_bias,
    const std::optional<torch::Tensor>& conv_state_indices,
    const std::optional<torch::Tensor>& ssm_state_indices, int32_t pad_slot_id,
    float softplus_beta, float softplus_threshold, bool use_qk_l2norm) {
  check_conv_decode(mixed_qkv, conv_state, conv_weight, ssm_state, num_heads_qk, num_heads_v,
                    head_k, head_v);
  const int64_t B = mixed_qkv.size(0);
  TORCH_CHECK(a.dim() == 2 && a.size(0) == B && a.size(1) == num_heads_v,
              "a must have shape [B, num_heads_v]");
  TORCH_CHECK(b.sizes() == a.sizes(), "a/b shape mismatch");
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "a and b must have the same dtype");
  TORCH_CHECK(A_log.scalar_type() == torch::kFloat32 && A_log.numel() == num_heads_v,
              "A_log must be float32 [num_heads_v]");
  TORCH_CHECK(dt_bias.scalar_type() == torch::kFloat32 && dt_bias.numel() == num_heads_v,
              "dt_bias must be float32 [num_heads_v]");
  const float sc = scale.has_value() ? *scale : 1.0f / std::sqrt(static_cast<float>(head_k));
  auto x = mixed_qkv.stride(1) == 1 ? mixed_qkv : mixed_qkv.contiguous();
  torch::Tensor cb, ci, si;
  if (has(conv_bias)) cb = conv_bias->to(conv_weight.scalar_type()).contiguous();
  if (has(conv_state_indices)) ci = conv_state_indices->to(torch::kInt32).contiguous();
  if (has(ssm_state_indices)) si = ssm_state_indices->to(torch::kInt32).contiguous();
  auto ac = a.contiguous(), bc = b.contiguous();
  auto al = A_log.contiguous(), db = dt_bias.contiguous();
  auto o = torch::empty({B, num_heads_v, head_v}, x.options());
  check(xk_gdn_conv_gating_decode(
            x.data_ptr(), x.stride(0), conv_state.data_ptr(), conv_state.stride(0),
            conv_state.stride(1), conv_state.stride(2), conv_state.size(0), conv_state.size(2),
            conv_weight.data_ptr(), conv_weight.stride(0), conv_weight.stride(1), ptr(cb),
            xdt(conv_weight), conv_weight.size(1), static_cast<const int32_t*>(ptr(ci)),
            pad_slot_id, static_cast<const float*>(al.data_ptr()), ac.data_ptr(),
            static_cast<const float*>(db.data_ptr()), bc.data_ptr(), xdt(ac), softplus_beta,
            softplus_threshold, static_cast<float*>(ssm_state.data_ptr()), ssm_state.stride(0),
            ssm_state.size(0), static_cast<const int32_t*>(ptr(si)), o.data_ptr(), B,
            num_heads_qk, num_heads_v, head_k, head_v, sc, use_qk_l2norm, xdt(x),
            stream_of(x)),
        "xk_gdn_conv_gating_decode");
  return o;
}

}  // namespace xllm::kernel::npu

namespace npu_ops {

// ascendc_npu/gemma_rms_norm.cpp:28-57
void npu_gemma_rms_norm(const torch::Tensor& x, const torch::Tensor& gamma, double epsilon,
                        torch::Tensor& rstdOut, torch::Tensor& yOut) {
  const int64_t dx = x.dim(), dg = gamma.dim(), N = gamma.numel();
  TORCH_CHECK(dx >= dg && x.sizes().slice(dx - dg) == gamma.sizes(),
              "gamma shape must match the trailing dims of x");
  std::vector<int64_t> rshape;
  if (dx > dg) {
    for (int64_t i = 0; i < dx - dg; ++i) rshape.push_back(x.size(i));
    for (int64_t i = 0; i < dg; ++i) rshape.push_back(1);
  } else {
    rshape.assign(dx, 1);
  }
  auto x2 = rows(x, N);
  auto y = torch::empty_like(x2);
  auto rstd = torch::empty(rshape, x.options().dtype(torch::kFloat32));
  auto gm = gamma.contiguous();
  check(xk_gemma_rms_norm(x2.data_ptr(), x2.stride(0), y.data_ptr(), y.stride(0), gm.data_ptr(),
                          static_cast<float*>(rstd.data_ptr()), x2.size(0), N,
                          static_cast<float>(epsilon), xdt(x), xdt(gm), stream_of(x)),
        "xk_gemma_rms_norm");
  yOut = y.reshape(x.sizes());
  rstdOut = rstd;
}

// ascendc_npu/layer_norm_fwd.cpp:24-80
torch::Tensor layer_norm_fwd(const torch::Tensor& x, const torch::Tensor& weight,
                             const c10::optional<torch::Tensor>& bias, double eps,
                             const c10::optional<torch::Tensor>& z, int64_t group_size,
                             bool norm_before_gate, bool is_rms_norm) {
  torch::Tensor b;
  if (bias.has_value() && bias->defined()) b = *bias;
  return layer_norm_impl(x, weight, b, eps, z, group_size, norm_before_gate, is_rms_norm);
}

}  // namespace npu_ops
