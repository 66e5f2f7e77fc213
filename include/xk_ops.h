/*
 * xk_ops.h -- C-ABI of the MI355X (gfx950) kernels behind the xLLM
 * Triton-Ascend op set (reference: Fengfengst123/torch_npu_ops, triton_npu/).
 *
 * This ABI replaces the reference's launch runtime: the `.npubin` loader
 * (triton_npu/kernel_registry.cpp:112-296), the packed-argument blob
 * (triton_npu/args_builder.h:34-302) and OperationBase::execute
 * (triton_npu/operation_base.h:136-192).  Every function here
 *   - takes raw device pointers, element strides, scalar parameters, dtype
 *     enums and a hipStream_t passed as `void*`;
 *   - returns 0 on success, a negative XK_ERR_* code for an argument the
 *     kernels cannot take, or a positive hipError_t for a launch failure;
 *   - never throws, never synchronises and never touches host memory;
 *   - allocates nothing: where a kernel needs scratch memory the caller
 *     passes a workspace whose size the matching *_workspace_bytes()
 *     function reports (this replaces the JSON `workspace_size` field,
 *     kernel_registry.cpp:55-107);
 *   - launches only on the stream it is given, so it is safe under
 *     hipGraph capture.
 * All tensors are row-major.  "stride" arguments count elements, not bytes.
 */
#ifndef XK_OPS_H_
#define XK_OPS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types understood by the kernels. */
typedef enum xk_dtype {
  XK_F32 = 0,
  XK_BF16 = 1,
  XK_F16 = 2,
  XK_I32 = 3,
  XK_I64 = 4
} xk_dtype;

/* Status codes (negative); positive values are hipError_t. */
#define XK_OK 0
#define XK_ERR_INVALID (-1)     /* shape / pointer / value the op rejects */
#define XK_ERR_UNSUPPORTED (-2) /* dtype or configuration not built */
#define XK_ERR_WORKSPACE (-3)   /* workspace missing or too small */
#define XK_ERR_SCRATCH (-4)     /* problem larger than the static scratch */

const char* xk_version(void);
const char* xk_status_string(int status);

/* ------------------------------------------------------------------------
 * Grouped LayerNorm / RMSNorm forward with optional SiLU gate.
 * Replaces xllm::kernel::npu::layer_norm_fwd
 *   (triton_npu/torch_api/triton_ops_api.h:137-145,
 *    npu_triton_layernorm_fwd.cpp:48-332)
 * and npu_ops::layer_norm_fwd (ascendc_npu/ascendc_ops_api.h:31-39).
 *   x, y, z : [M, N] rows with row strides; dtype `dtype` (f32/bf16/f16).
 *   weight, bias : [N], dtype `wdtype`; bias and z may be NULL.
 *   mean, rstd : fp32 [ngroups * M] at index group * M + row; mean is
 *     ignored (may be NULL) when is_rms_norm, either may be NULL.
 *   group_size divides N.  gate = z * sigmoid(z) is applied to y
 *   (norm_before_gate != 0) or to x before the statistics.
 */
int xk_layer_norm_fwd(const void* x, int64_t stride_x_row, void* y,
                      int64_t stride_y_row, const void* weight,
                      const void* bias, const void* z, int64_t stride_z_row,
                      float* mean, float* rstd, int64_t M, int64_t N,
                      int64_t group_size, float eps, int norm_before_gate,
                      int is_rms_norm, xk_dtype dtype, xk_dtype wdtype,
                      void* stream);

/* ------------------------------------------------------------------------
 * Gemma RMSNorm: y = x * rsqrt(mean(x^2) + eps) * (1 + gamma), fp32
 * arithmetic, one statistic per row of N = gamma.numel() elements.
 * Replaces npu_ops::npu_gemma_rms_norm (ascendc_npu/ascendc_ops_api.h:24-29,
 * gemma_rms_norm.cpp:28-57).  rstd: fp32 [M] (may be NULL).
 */
int xk_gemma_rms_norm(const void* x, int64_t stride_x_row, void* y,
                      int64_t stride_y_row, const void* gamma, float* rstd,
                      int64_t M, int64_t N, float eps, xk_dtype dtype,
                      xk_dtype wdtype, void* stream);

/* ------------------------------------------------------------------------
 * y = x * rsqrt(sum(x^2) + eps) over the last dim (contiguous rows).
 * Replaces npu_l2norm_last_dim (triton_ops_api.h:31, npu_triton_l2norm.cpp).
 */
int xk_l2norm_last_dim(const void* x, void* y, int64_t rows, int64_t cols,
                       float eps, xk_dtype dtype, xk_dtype out_dtype,
                       void* stream);

/* ------------------------------------------------------------------------
 * Split a packed [T, q_hidden + 2*kv_hidden] row into q, k, v; per-head
 * RMSNorm of q and k (x * 1/sqrt(mean(x^2)+eps) * w (+ b)) followed by neox
 * rotate-half RoPE over the whole head; v copied through.
 * Replaces xllm::kernel::npu::npu_split_rmsnorm_rope
 *   (triton_npu/torch_api/triton_ops_api.h:186-198,
 *    npu_triton_split_rmsnorm_rope.cpp:56-144).
 *   cos/sin : [T, head_dim] rows (stride_sc_row), dtype aux_dtype; or, when
 *     `positions` (int32/int64 [T]) is given, computed in registers as
 *     cos/sin(pos * inv_freq[d mod head_dim/2]) from the fp32 table
 *     inv_freq[head_dim/2] (sin/cos pointers then ignored).
 *   q_weight, k_weight (+ optional biases): [head_dim], dtype aux_dtype.
 *   q_out [T, q_hidden], k_out / v_out [T, kv_hidden], dtype `dtype`.
 *   aux_dtype is `dtype` or XK_F32; head_dim is 64, 128 or 256.
 */
int xk_split_rmsnorm_rope(const void* qkv, int64_t stride_qkv_row,
                          int64_t num_tokens, const void* sin,
                          const void* cos, int64_t stride_sc_row,
                          const void* positions, xk_dtype pos_dtype,
                          const float* inv_freq, void* q_out, void* k_out,
                          void* v_out, const void* q_weight,
                          const void* q_bias, const void* k_weight,
                          const void* k_bias, xk_dtype aux_dtype,
                          int64_t q_hidden, int64_t kv_hidden,
                          int64_t head_dim, float eps, xk_dtype dtype,
                          void* stream);

/* ------------------------------------------------------------------------
 * In-place GPT-J (interleaved) RoPE on the last rope_dim elements of rows.
 * Replaces xllm::kernel::npu::rope_inplace
 *   (triton_npu/torch_api/triton_ops_api.h:68-71,
 *    npu_triton_rope_inplace.cpp:22-64; kernel
 *    triton_src/test_rope_inplace.py:17-49).
 *   x : rows of `hidden` elements (row stride stride_x_row), updated in
 *   place; row r uses sin / cos row r / head_num ([*, >= rope_dim], row stride
 *   stride_sc_row, in sc_dtype = dtype or fp32).  With d = hidden - rope_dim:
 *     x[d+2i]   <- x[d+2i] cos[2i] - x[d+2i+1] sin[2i]
 *     x[d+2i+1] <- x[d+2i+1] cos[2i+1] + x[d+2i] sin[2i+1]
 *   rope_dim even; offsets and strides even.
 */
int xk_rope_inplace(void* x, int64_t rows, int64_t head_num, int64_t stride_x_row,
                    int64_t hidden, const void* sin, const void* cos,
                    int64_t stride_sc_row, int64_t rope_dim, xk_dtype dtype,
                    xk_dtype sc_dtype, void* stream);

/* ------------------------------------------------------------------------
 * Depthwise causal conv1d state update (decode / short MTP windows).
 * Replaces xllm::kernel::npu::npu_causal_conv1d_update
 *   (triton_npu/torch_api/triton_ops_api.h:147-160,
 *    npu_triton_causal_conv1d_update.cpp:22-138).
 *   x, out : [batch, dim, seqlen] (strides); conv_state : [lines, dim,
 *   state_len] (strides), updated in place to the last state_len entries of
 *   cat(state, x); weight [dim, width] (strides), bias [dim] or NULL, both
 *   dtype wdtype (x's dtype or fp32).  Slot b = conv_state_indices[b] (or b
 *   when NULL); slots equal to pad_slot_id or outside [0, num_cache_lines)
 *   are skipped (no output, no state write).  activation != 0 applies SiLU.
 *   state_len >= width - 1.
 */
int xk_causal_conv1d_update(
    const void* x, int64_t stride_x_batch, int64_t stride_x_dim,
    int64_t stride_x_token, void* conv_state, int64_t stride_state_line,
    int64_t stride_state_dim, int64_t stride_state_token,
    const void* weight, int64_t stride_w_dim, int64_t stride_w_tap,
    const void* bias, xk_dtype wdtype, const int32_t* conv_state_indices,
    int32_t pad_slot_id, int64_t num_cache_lines, void* out,
    int64_t stride_o_batch, int64_t stride_o_dim, int64_t stride_o_token,
    int64_t batch, int64_t dim, int64_t seqlen, int64_t width,
    int64_t state_len, int activation, xk_dtype dtype, void* stream);

/* ------------------------------------------------------------------------
 * Varlen depthwise causal conv1d with conv-state slots (prefill, APC,
 * speculative decoding).
 * Replaces xllm::kernel::npu::npu_causal_conv1d_update_v2
 *   (triton_npu/torch_api/triton_ops_api.h:162-176,
 *    npu_triton_causal_conv1d_update_v2.cpp:99-239).
 *   x, out : [num_tokens, dim] token-major (token strides); sequence s is
 *     rows [query_start_loc[s], query_start_loc[s+1]), s < batch.
 *   conv_state : [num_cache_lines, dim, state_len] (strides).
 *   slot_table : NULL (slot = s), 1-D [batch] (slot_table_2d = 0) or 2-D
 *     [batch, slot_table_stride] whose columns initial_state_idx[s] /
 *     last_state_idx[s] (NULL = column 0) give the input / output slot.
 *   num_accepted_tokens : NULL, or [batch] for speculative decoding.
 *   state_rule 0 reproduces the reference's final-state rule
 *     (state_len_run = eff - (max_query_len - len)); 1 keeps the last
 *     eff = width-1 (+ max_query_len-1 with spec decoding) inputs of every
 *     sequence.  Sequences whose input slot is pad_slot_id are skipped.
 *   width in [1, 8]; one kernel (the lane that reads a sequence's history
 *   writes its final state).  A sequence's input slot must not be another
 *   sequence's output slot in the same call.
 */
int xk_causal_conv1d_varlen(
    const void* x, int64_t stride_x_token, int64_t num_tokens, void* out,
    int64_t stride_o_token, void* conv_state, int64_t stride_state_line,
    int64_t stride_state_dim, int64_t stride_state_token,
    int64_t num_cache_lines, int64_t state_len, const void* weight,
    int64_t stride_w_dim, int64_t stride_w_tap, const void* bias,
    xk_dtype wdtype, const int32_t* query_start_loc, int64_t batch,
    const int32_t* slot_table, int64_t slot_table_stride, int slot_table_2d,
    const int32_t* initial_state_idx, const int32_t* last_state_idx,
    const int32_t* num_accepted_tokens, int64_t dim, int64_t width,
    int64_t max_query_len, int state_rule, int activation,
    int32_t pad_slot_id, xk_dtype dtype, void* stream);

/* ------------------------------------------------------------------------
 * Gated delta rule, recurrent form (decode, speculative windows).
 * Replaces xllm::kernel::npu::npu_fused_recurrent_gated_delta_rule
 *   (triton_npu/torch_api/triton_ops_api.h:81-93,
 *    npu_triton_recurrent_gated_delta_rule.cpp:54-247).
 *   q, k : [tokens, H, K]; v, o : [tokens, HV, V] (dtype); g, beta :
 *   [tokens, HV] (g_dtype / beta_dtype; beta NULL = 1).  Sequences are
 *   cu_seqlens[n]..cu_seqlens[n+1] (int32/int64) or, when NULL, N runs of T
 *   tokens.  States are fp32 [*, HV, K, V]: the initial state of sequence n
 *   is initial_state[slot] with slot = ssm_state_indices[n*stride_idx_seq +
 *   c*stride_idx_tok] (c = num_accepted_tokens[n]-1 with speculative
 *   decoding, else 0; slot = n without indices); out-of-range slots start
 *   from zero and are not written.  inplace_final_state != 0 writes the
 *   state into final_state (normally == initial_state) at that slot, or
 *   after every token t at column t when stride_idx_tok != 0; otherwise
 *   final_state is a dense [N, HV, K, V].  use_qk_l2norm normalises q and k
 *   by 1/sqrt(sum^2 + 1e-6) before `scale`.  (K, V) in {64, 128}^2.
 */
int xk_gdn_recurrent(
    const void* q, const void* k, const void* v, xk_dtype dtype, const void* g,
    xk_dtype g_dtype, const void* beta, xk_dtype beta_dtype, void* o,
    const float* initial_state, int64_t stride_h0_slot, float* final_state,
    int64_t stride_ht_slot, int64_t num_slots, const void* cu_seqlens,
    xk_dtype cu_dtype, const int32_t* ssm_state_indices, int64_t stride_idx_seq,
    int64_t stride_idx_tok, const int32_t* num_accepted_tokens, int64_t N,
    int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
    int use_qk_l2norm, int inplace_final_state, void* stream);

/* ------------------------------------------------------------------------
 * GDN gating (the step before both gated-delta-rule forms).
 * Replaces xllm::kernel::npu::npu_fused_gdn_gating
 *   (triton_npu/torch_api/triton_ops_api.h:73-79,
 *    npu_triton_fused_gdn_gating.cpp:33-94; kernel
 *    triton_src/test_fused_gdn_gating.py:10-43).
 *   For rows x heads (a, b [rows, heads] in ab_dtype; A_log, dt_bias fp32
 *   [heads]):
 *     x        = a + dt_bias
 *     g        = -exp(A_log) * (softplus_beta * x <= threshold
 *                               ? log(1 + exp(softplus_beta * x)) / softplus_beta
 *                               : x)                        (fp32 [rows, heads])
 *     beta_out = sigmoid(b)                                  (ab_dtype)
 */
int xk_fused_gdn_gating(const float* A_log, const void* a, const void* b,
                        const float* dt_bias, float* g_out, void* beta_out,
                        int64_t rows, int64_t heads, float softplus_beta,
                        float threshold, xk_dtype ab_dtype, void* stream);

/* ------------------------------------------------------------------------
 * Recurrent gated delta rule with the gating computed in the kernel.
 * Replaces xllm::kernel::npu::npu_fused_sigmoid_gating_delta_rule_update
 *   (triton_npu/torch_api/triton_ops_api.h:95-109,
 *    npu_triton_fused_sigmoid_gating_delta_rule_update.cpp:54-177; kernel
 *    triton_src/test_fused_sigmoid_gating_delta_rule_update.py:10-117).
 *   Per token, g and beta come from a and b ([tokens, HV], ab_dtype) as in
 *   xk_fused_gdn_gating; then the recurrent step of xk_gdn_recurrent runs.
 *   Sequences are cu_seqlens[n]..cu_seqlens[n+1] (int32).  The state pool
 *   state [num_slots, HV, K, V] (fp32) is updated in place: sequence n
 *   starts from state[state_indices[n]] and writes its final state there; a
 *   negative (or out-of-range) index starts from zeros and writes nothing.
 *   o : [tokens, HV, V] in dtype.  use_qk_l2norm normalises q and k by
 *   1/sqrt(sum^2 + 1e-6) before `scale`.  (K, V) in {64, 128}^2.
 */
int xk_gdn_sigmoid_gating_update(
    const float* A_log, const void* a, const float* dt_bias, float softplus_beta,
    float threshold, const void* q, const void* k, const void* v, const void* b,
    xk_dtype ab_dtype, void* o, float* state, int64_t stride_state_slot,
    int64_t num_slots, const int32_t* state_indices, const int32_t* cu_seqlens,
    int64_t N, int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
    int use_qk_l2norm, xk_dtype dtype, void* stream);

/* ------------------------------------------------------------------------
 * Split of the GDN input projection (the step before the conv1d).
 * Replaces xllm::kernel::npu::npu_fused_qkvzba_split_reshape_cat
 *   (triton_npu/torch_api/triton_ops_api.h:178-184,
 *    npu_triton_fused_qkvzba_split_reshape.cpp:116-230; kernels
 *    triton_src/test_fused_qkvzba_split_reshape.py:31-351).
 *   R = num_heads_v / num_heads_qk.  Each row of mixed_qkvz holds
 *   num_heads_qk groups [q (head_qk) | k (head_qk) | v (R*head_v) |
 *   z (R*head_v)]; each row of mixed_ba holds groups [b (R) | a (R)].
 *   Outputs (dense rows): mixed_qkv [rows, 2*num_heads_qk*head_qk +
 *   num_heads_v*head_v] = [all q | all k | all v], z [rows, num_heads_v *
 *   head_v], b and a [rows, num_heads_v].  A permutation: exact copies.
 */
int xk_fused_qkvzba_split_reshape_cat(
    const void* mixed_qkvz, int64_t stride_qkvz_row, const void* mixed_ba,
    int64_t stride_ba_row, void* mixed_qkv, void* z, void* b, void* a, int64_t rows,
    int64_t num_heads_qk, int64_t num_heads_v, int64_t head_qk, int64_t head_v,
    xk_dtype dtype, xk_dtype ba_dtype, void* stream);

/* ------------------------------------------------------------------------
 * One decode step of the gated delta rule fused with the causal conv1d
 * update of its mixed q/k/v projection (no single reference function: the
 * composition of npu_causal_conv1d_update, the [q | k | v] channel split of
 * triton_npu/triton_src/test_fused_qkvzba_split_reshape.py:493-500 and
 * npu_fused_recurrent_gated_delta_rule).
 *   mixed_qkv : [B, 2*H*K + HV*V] (row stride), conv over the state
 *   [lines, D, conv_state_len] with weight [D, width] (+ bias) and SiLU, the
 *   state shifted in place; then q = ch[0:H*K], k = ch[H*K:2*H*K],
 *   v = ch[2*H*K:], l2norm (optional) and one GDN step on
 *   ssm_state[ssm_state_indices[b]] (fp32 [slots, HV, K, V], in place).
 *   g, beta : [B, HV].  o : [B, HV, V].  Rows whose conv slot equals
 *   pad_slot_id are skipped.  K = V = 128, HV/H <= 16.
 */
int xk_gdn_conv_decode(
    const void* mixed_qkv, int64_t stride_x_row, void* conv_state,
    int64_t stride_cs_line, int64_t stride_cs_dim, int64_t stride_cs_tok,
    int64_t conv_lines, int64_t conv_state_len, const void* conv_weight,
    int64_t stride_w_dim, int64_t stride_w_tap, const void* conv_bias,
    xk_dtype w_dtype, int64_t width, const int32_t* conv_state_indices,
    int32_t pad_slot_id, const void* g, xk_dtype g_dtype, const void* beta,
    xk_dtype beta_dtype, float* ssm_state, int64_t stride_state_slot,
    int64_t num_slots, const int32_t* ssm_state_indices, void* o, int64_t B,
    int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
    int use_qk_l2norm, xk_dtype dtype, void* stream);

/* ------------------------------------------------------------------------
 * xk_gdn_conv_decode with the GDN gating computed in the kernel (the decode
 * step from the projection outputs in one launch): per (row, v head) the
 * log-decay g = -exp(A_log) * softplus_{softplus_beta, threshold}(a +
 * dt_bias) and beta = sigmoid(b), in fp32 registers, as
 * xk_gdn_sigmoid_gating_update forms them (reference pair:
 * npu_triton_fused_sigmoid_gating_delta_rule_update.cpp:54-177 after
 * npu_causal_conv1d_update).  a, b : [B, HV] in ab_dtype; A_log, dt_bias :
 * fp32 [HV].  Every other argument as xk_gdn_conv_decode; a state index
 * outside [0, num_slots) starts from a zero state and writes nothing.
 */
int xk_gdn_conv_gating_decode(
    const void* mixed_qkv, int64_t stride_x_row, void* conv_state,
    int64_t stride_cs_line, int64_t stride_cs_dim, int64_t stride_cs_tok,
    int64_t conv_lines, int64_t conv_state_len, const void* conv_weight,
    int64_t stride_w_dim, int64_t stride_w_tap, const void* conv_bias,
    xk_dtype w_dtype, int64_t width, const int32_t* conv_state_indices,
    int32_t pad_slot_id, const float* A_log, const void* a, const float* dt_bias,
    const void* b, xk_dtype ab_dtype, float softplus_beta, float threshold,
    float* ssm_state, int64_t stride_state_slot, int64_t num_slots,
    const int32_t* ssm_state_indices, void* o, int64_t B, int64_t H, int64_t HV,
    int64_t K, int64_t V, float scale, int use_qk_l2norm, xk_dtype dtype,
    void* stream);

/* ------------------------------------------------------------------------
 * Chunked gated delta rule (prefill), chunk size 64.
 * Replaces xllm::kernel::npu::npu_chunk_gated_delta_rule
 *   (triton_npu/torch_api/triton_ops_api.h:111-122,
 *    npu_triton_chunk_gated_delta_rule.cpp:556-642) -- the whole pipeline
 * of cumsum, scaled K K^T, solve_tril, WY recompute, state recurrence and
 * output (a6b-a6g) in three launches with no host synchronisation.
 *   q, k : [total_tokens, H, K]; v, o : [total_tokens, HV, V] (dtype
 *   bf16, as the reference requires); g : [total_tokens, HV] log-decay,
 *   beta : [total_tokens, HV] (each fp32 or bf16); sequences
 *   cu_seqlens[n]..cu_seqlens[n+1] (int32 or int64, device).
 *   initial_state / final_state : fp32 [N, HV, K, V] (NULL = zero / not
 *   written).  use_qk_l2norm applies x / sqrt(sum x^2 + 1e-6) to q and k
 *   first.  K = 128, V a multiple of 32.  q, k, v 16-byte aligned, o
 *   8-byte aligned (else XK_ERR_INVALID).
 *   workspace >= xk_gdn_chunk_workspace_bytes(total_tokens, N, HV) bytes,
 *   256-byte aligned (chunk offsets + per-chunk inverse blocks).
 */
int64_t xk_gdn_chunk_workspace_bytes(int64_t total_tokens, int64_t num_seqs,
                                     int64_t HV);
int xk_gdn_chunk_fwd(
    const void* q, const void* k, const void* v, xk_dtype dtype, const void* g,
    xk_dtype g_dtype, const void* beta, xk_dtype beta_dtype, void* o,
    const float* initial_state, float* final_state, const void* cu_seqlens,
    xk_dtype cu_dtype, int64_t N, int64_t total_tokens, int64_t H, int64_t HV,
    int64_t K, int64_t V, float scale, int use_qk_l2norm, void* workspace,
    size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * xk_gdn_chunk_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * Same arguments and results as xk_gdn_chunk_fwd (the same kernels run);
 * the workspace is a static device buffer of 64 MiB that the library holds
 * on every GPU it runs on until the process ends.  Calls whose
 * xk_gdn_chunk_workspace_bytes(total_tokens, N, HV) exceeds 64 MiB return
 * XK_ERR_SCRATCH (e.g. up to ~6,700 tokens at HV = 32, ~27,000 at HV = 8).
 * The call allocates nothing; `stream` must belong to the current device.
 * Every call on one GPU shares that GPU's buffer: calls that overlap in
 * time on one GPU (other streams, other host threads) race.
 */
int xk_gdn_chunk_fwd_noalloc(
    const void* q, const void* k, const void* v, xk_dtype dtype, const void* g,
    xk_dtype g_dtype, const void* beta, xk_dtype beta_dtype, void* o,
    const float* initial_state, float* final_state, const void* cu_seqlens,
    xk_dtype cu_dtype, int64_t N, int64_t total_tokens, int64_t H, int64_t HV,
    int64_t K, int64_t V, float scale, int use_qk_l2norm, void* stream);

/*
 * The chunked pipeline stage by stage, in the reference's
 * intermediate layouts (chunk size 64; chunks restart at every sequence):
 *   g, g_cumsum, beta [T, H]; q, k [T, Hg, K]; v, u, v_new, o [T, H, V];
 *   A, Ai [T, H, 64] (row t: row t - chunk start of the chunk's matrix);
 *   w [T, H, K]; h [num_chunks, H, K, V] (chunks of all sequences in order).
 * T = total_tokens; sequences by cu_seqlens (int32/int64, N + 1 entries,
 * device).  K = 128 (V = 128 for w_u and fwd_o, a multiple of 32 for
 * fwd_h); q/k/v/w/u/h bf16.  Decays are exp(x) for x <= 0, else 0.
 * Except for the cumsum, every stage needs a workspace of
 * xk_gdn_stage_workspace_bytes(N) bytes, 256-byte aligned.
 */
int64_t xk_gdn_stage_workspace_bytes(int64_t num_seqs);

/* Per-chunk inclusive cumsum of g (fp32/bf16/f16) into fp32 out
 * [T, H]; chunk_size a power of two.  Replaces npu_chunk_local_cumsum
 * (triton_ops_api.h:34-37, npu_triton_chunk_gated_delta_rule.cpp:151-227);
 * tokens outside every sequence get 0. */
int xk_chunk_local_cumsum(const void* g, xk_dtype g_dtype, float* out,
                          int64_t total_tokens, int64_t H,
                          const void* cu_seqlens, xk_dtype cu_dtype, int64_t N,
                          int64_t chunk_size, void* stream);

/* A = strict_tril(beta_i (k_i . k_j) exp(gc_i - gc_j)), fp32 [T, H, 64];
 * g_cumsum NULL = no decay.  Replaces npu_chunk_scaled_dot_kkt_fwd
 * (triton_ops_api.h:39-44, npu_triton_chunk_gated_delta_rule.cpp:229-297). */
int xk_chunk_scaled_dot_kkt(const void* k, xk_dtype dtype, const void* beta,
                            xk_dtype beta_dtype, const float* g_cumsum,
                            float* A, int64_t total_tokens, int64_t Hg,
                            int64_t H, int64_t K, const void* cu_seqlens,
                            xk_dtype cu_dtype, int64_t N, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Ai = (I + A)^-1 per chunk (only the strictly lower part of A is read),
 * written in ai_dtype (f32/bf16/f16).  Replaces npu_solve_tril
 * (triton_ops_api.h:46-49, npu_triton_chunk_gated_delta_rule.cpp:299-395). */
int xk_solve_tril(const float* A, void* Ai, xk_dtype ai_dtype,
                  int64_t total_tokens, int64_t H, const void* cu_seqlens,
                  xk_dtype cu_dtype, int64_t N, void* workspace,
                  size_t workspace_bytes, void* stream);

/* u = Ai (v beta), w = Ai (k beta exp(gc)); Ai bf16 or fp32, outputs bf16.
 * k, v, Ai, w and u 16-byte aligned (else XK_ERR_INVALID).  Replaces npu_recompute_w_u_fwd (triton_ops_api.h:51-57,
 * npu_triton_chunk_gated_delta_rule.cpp:397-475). */
int xk_recompute_w_u(const void* k, const void* v, xk_dtype dtype,
                     const void* beta, xk_dtype beta_dtype,
                     const float* g_cumsum, const void* Ai, xk_dtype ai_dtype,
                     void* w, void* u, int64_t total_tokens, int64_t Hg,
                     int64_t H, int64_t K, int64_t V, const void* cu_seqlens,
                     xk_dtype cu_dtype, int64_t N, void* workspace,
                     size_t workspace_bytes, void* stream);

/* The state recurrence: per chunk c, h[c] = state entering the chunk (bf16),
 * v_new = u - w S (bf16, NULL = not stored), S <- exp(gc_last) S +
 * k^T (v_new exp(gc_last - gc)); final_state fp32 [N, H, K, V] (NULL = not
 * written); initial_state fp32 or NULL; g_cumsum NULL = no decay.  h holds
 * num_chunks chunks.  Replaces npu_chunk_gated_delta_rule_fwd_h
 * (triton_ops_api.h:124-135, npu_triton_chunk_gated_delta_rule.cpp:644-802). */
int xk_chunk_fwd_h(const void* k, const void* w, const void* u, xk_dtype dtype,
                   const float* g_cumsum, const float* initial_state, void* h,
                   int64_t num_chunks, void* v_new, float* final_state,
                   int64_t total_tokens, int64_t Hg, int64_t H, int64_t K,
                   int64_t V, const void* cu_seqlens, xk_dtype cu_dtype,
                   int64_t N, void* workspace, size_t workspace_bytes,
                   void* stream);

/* o = scale (exp(gc) (q h[c]) + tril(q k^T exp(gc_i - gc_j)) v), with the
 * masked q k^T rounded to bf16 before the product as the reference does.
 * Replaces npu_chunk_fwd_o (triton_ops_api.h:59-66,
 * npu_triton_chunk_gated_delta_rule.cpp:477-554). */
int xk_chunk_fwd_o(const void* q, const void* k, const void* v, const void* h,
                   int64_t num_chunks, xk_dtype dtype, const float* g_cumsum,
                   void* o, float scale, int64_t total_tokens, int64_t Hg,
                   int64_t H, int64_t K, int64_t V, const void* cu_seqlens,
                   xk_dtype cu_dtype, int64_t N, void* workspace,
                   size_t workspace_bytes, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* XK_OPS_H_ */
