"""Python view of the op set over the C-ABI (tests, bench, smoke).

Each function here validates like the reference's torch_api wrapper it
mirrors (the file:line is in its docstring), allocates outputs with torch on
the input's device, and launches the HIP kernel through libxk.so on torch's
current stream.  There is no CPU path: a tensor that is not on a GPU, or a
missing libxk.so, raises.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from ._lib import check, lib

_DT = {
    torch.float32: _lib.XK_F32,
    torch.bfloat16: _lib.XK_BF16,
    torch.float16: _lib.XK_F16,
    torch.int32: _lib.XK_I32,
    torch.int64: _lib.XK_I64,
}


def xk_dtype(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _stream(t: torch.Tensor) -> int:
    if not t.is_cuda:
        raise RuntimeError("torch_npu_ops_amd ops need tensors on a GPU device")
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# Normalisation
# ---------------------------------------------------------------------------
def layer_norm_fwd(x: torch.Tensor, weight: torch.Tensor,
                   bias: Optional[torch.Tensor], eps: float,
                   z: Optional[torch.Tensor] = None, group_size: int = -1,
                   norm_before_gate: bool = True, is_rms_norm: bool = False,
                   return_stats: bool = False):
    """Grouped LayerNorm/RMSNorm with optional gate.

    Mirrors xllm::kernel::npu::layer_norm_fwd
    (triton_npu/torch_api/npu_triton_layernorm_fwd.cpp:48-332) and
    npu_ops::layer_norm_fwd (ascendc_npu/layer_norm_fwd.cpp:24-80): returns
    y shaped like x; with ``return_stats`` also the fp32 mean (None for RMS)
    and rstd of length ngroups * M at index group * M + row.
    """
    if x.dim() < 1:
        raise ValueError("layer_norm_fwd expects x.dim() >= 1")
    N = x.size(-1)
    G = group_size if group_size > 0 else N
    if N % G != 0:
        raise ValueError("x.size(-1) must be divisible by group_size")
    if weight.numel() != N:
        raise ValueError("weight numel must equal x.size(-1)")
    if bias is not None and bias.numel() != N:
        raise ValueError("bias numel must equal x.size(-1)")
    x2 = x.reshape(-1, N)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    z2 = None
    if z is not None:
        if z.shape != x.shape:
            raise ValueError("z shape must match x shape")
        z2 = z.reshape(-1, N)
        if z2.stride(-1) != 1:
            z2 = z2.contiguous()
    M = x2.size(0)
    weight = weight.contiguous()
    if bias is not None:
        bias = bias.contiguous().to(weight.dtype)
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    ng = N // G
    mean = None if is_rms_norm else torch.empty(ng * M, dtype=torch.float32,
                                                device=x.device)
    rstd = torch.empty(ng * M, dtype=torch.float32, device=x.device)
    st = lib().xk_layer_norm_fwd(
        x2.data_ptr(), x2.stride(0), y.data_ptr(), y.stride(0),
        weight.data_ptr(), _ptr(bias), _ptr(z2),
        z2.stride(0) if z2 is not None else 0, _ptr(mean), rstd.data_ptr(),
        M, N, G, float(eps), int(norm_before_gate), int(is_rms_norm),
        xk_dtype(x), xk_dtype(weight), _stream(x))
    check(st, "xk_layer_norm_fwd")
    y = y.reshape(x.shape)
    if return_stats:
        return y, mean, rstd
    return y


def npu_gemma_rms_norm(x: torch.Tensor, gamma: torch.Tensor, epsilon: float):
    """y = x * rsqrt(mean(x^2) + eps) * (1 + gamma); returns (y, rstd).

    Mirrors npu_ops::npu_gemma_rms_norm (ascendc_npu/gemma_rms_norm.cpp:28-57):
    rstd has x's leading dims followed by gamma.dim() ones.
    """
    dg = gamma.dim()
    N = gamma.numel()
    if x.dim() < dg or tuple(x.shape[x.dim() - dg:]) != tuple(gamma.shape):
        raise ValueError("gamma shape must match the trailing dims of x")
    x2 = x.reshape(-1, N)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.size(0)
    lead = list(x.shape[: x.dim() - dg])
    rstd_shape = lead + [1] * dg if x.dim() > dg else [1] * x.dim()
    y = torch.empty_like(x2)
    rstd = torch.empty(rstd_shape, dtype=torch.float32, device=x.device)
    gamma = gamma.contiguous()
    st = lib().xk_gemma_rms_norm(
        x2.data_ptr(), x2.stride(0), y.data_ptr(), y.stride(0),
        gamma.data_ptr(), rstd.data_ptr(), M, N, float(epsilon),
        xk_dtype(x), xk_dtype(gamma), _stream(x))
    check(st, "xk_gemma_rms_norm")
    return y.reshape(x.shape), rstd


def npu_split_rmsnorm_rope(input: torch.Tensor, sin: Optional[torch.Tensor],
                           cos: Optional[torch.Tensor], q_weight: torch.Tensor,
                           k_weight: torch.Tensor, q_hidden_size: int,
                           kv_hidden_size: int, head_dim: int, eps: float,
                           q_bias: Optional[torch.Tensor] = None,
                           k_bias: Optional[torch.Tensor] = None,
                           bias: bool = False,
                           positions: Optional[torch.Tensor] = None,
                           inv_freq: Optional[torch.Tensor] = None):
    """Split + q/k RMSNorm + neox RoPE; returns (q, k, v).

    Mirrors npu_split_rmsnorm_rope
    (triton_npu/torch_api/npu_triton_split_rmsnorm_rope.cpp:56-144),
    including its shape checks; biases are used only when ``bias`` is set
    and both tensors are given (:109-118).  With ``positions`` (and an fp32
    ``inv_freq`` [head_dim/2]) cos/sin are computed in the kernel and the
    sin/cos arguments may be None.  The reference's launch-shape constraint
    (32 % n_kv_heads == 0, :94-96) does not apply to this kernel.
    """
    if input.dim() != 2:
        raise ValueError("split_rmsnorm_rope input must be a 2D tensor")
    if head_dim <= 0 or head_dim & (head_dim - 1):
        raise ValueError("split_rmsnorm_rope head_dim must be a power of two")
    if q_hidden_size % kv_hidden_size:
        raise ValueError("split_rmsnorm_rope q_hidden_size must be divisible "
                         "by kv_hidden_size")
    if kv_hidden_size % head_dim:
        raise ValueError("split_rmsnorm_rope kv_hidden_size must be divisible "
                         "by head_dim")
    if input.size(1) != q_hidden_size + 2 * kv_hidden_size:
        raise ValueError("split_rmsnorm_rope input hidden size mismatch")
    if q_weight.numel() != head_dim or k_weight.numel() != head_dim:
        raise ValueError("split_rmsnorm_rope q/k weight shape mismatch")
    T = input.size(0)
    x = input if input.stride(1) == 1 else input.contiguous()
    aux = q_weight.dtype
    qw, kw = q_weight.contiguous(), k_weight.contiguous().to(aux)
    qb = kb = None
    if bias and q_bias is not None and k_bias is not None:
        qb, kb = q_bias.contiguous().to(aux), k_bias.contiguous().to(aux)
    pos_ptr, pos_dt, inv_ptr = None, _lib.XK_I64, None
    sin_ptr = cos_ptr = None
    stride_sc = head_dim
    if positions is not None:
        if inv_freq is None or inv_freq.numel() != head_dim // 2:
            raise ValueError("positions mode needs inv_freq of head_dim/2 fp32")
        positions = positions.contiguous()
        inv_freq = inv_freq.to(torch.float32).contiguous()
        pos_ptr, pos_dt, inv_ptr = positions.data_ptr(), xk_dtype(positions), inv_freq.data_ptr()
    else:
        if (sin.dim() != 2 or cos.dim() != 2 or sin.size(0) != T or cos.size(0) != T
                or sin.size(1) != head_dim or cos.size(1) != head_dim):
            raise ValueError("split_rmsnorm_rope sin/cos shape mismatch")
        sin = sin.to(aux).contiguous()
        cos = cos.to(aux).contiguous()
        sin_ptr, cos_ptr = sin.data_ptr(), cos.data_ptr()
    q = torch.empty((T, q_hidden_size), dtype=input.dtype, device=input.device)
    k = torch.empty((T, kv_hidden_size), dtype=input.dtype, device=input.device)
    v = torch.empty((T, kv_hidden_size), dtype=input.dtype, device=input.device)
    st = lib().xk_split_rmsnorm_rope(
        x.data_ptr(), x.stride(0), T, sin_ptr, cos_ptr, stride_sc, pos_ptr,
        pos_dt, inv_ptr, q.data_ptr(), k.data_ptr(), v.data_ptr(), qw.data_ptr(),
        _ptr(qb), kw.data_ptr(), _ptr(kb), xk_dtype(qw), q_hidden_size,
        kv_hidden_size, head_dim, float(eps), xk_dtype(x), _stream(input))
    check(st, "xk_split_rmsnorm_rope")
    return q, k, v


def rope_inplace(x: torch.Tensor, sin: torch.Tensor, cos: torch.Tensor,
                 rope_dim: int = 64) -> torch.Tensor:
    """In-place GPT-J (interleaved) RoPE on the last rope_dim elements of
    each row of x ([bsz, hidden] or [bsz, heads, hidden]); sin / cos are
    [bsz, >= rope_dim].  Returns x.

    Mirrors rope_inplace (triton_npu/torch_api/npu_triton_rope_inplace.cpp:22-64).
    """
    if x.dim() == 2:
        bsz, heads, hidden = x.size(0), 1, x.size(1)
        x2 = x
    elif x.dim() == 3:
        bsz, heads, hidden = x.shape
        x2 = x.view(-1, hidden)
    else:
        raise ValueError(f"Unsupported dimension: {x.dim()}")
    if x2.stride(-1) != 1:
        raise ValueError("rope_inplace needs rows with unit column stride")
    if sin.stride(-1) != 1 or cos.stride(-1) != 1 or sin.stride(0) != cos.stride(0):
        raise ValueError("sin and cos must share a row stride with unit column stride")
    st = lib().xk_rope_inplace(x2.data_ptr(), bsz * heads, heads, x2.stride(0), hidden,
                               sin.data_ptr(), cos.data_ptr(), cos.stride(0), rope_dim,
                               xk_dtype(x2), xk_dtype(sin), _stream(x))
    check(st, "xk_rope_inplace")
    return x


def npu_causal_conv1d_update(x: torch.Tensor, conv_state: torch.Tensor,
                             weight: torch.Tensor, activation: bool = True,
                             bias: Optional[torch.Tensor] = None,
                             cache_seqlens: Optional[torch.Tensor] = None,
                             conv_state_indices: Optional[torch.Tensor] = None,
                             num_accepted_tokens: Optional[torch.Tensor] = None,
                             query_start_loc: Optional[torch.Tensor] = None,
                             max_query_len: int = -1,
                             intermediate_conv_window: Optional[torch.Tensor] = None,
                             pad_slot_id: int = -1, validate_data: bool = False):
    """Causal conv1d state update; conv_state is updated in place.

    Mirrors npu_causal_conv1d_update
    (triton_npu/torch_api/npu_triton_causal_conv1d_update.cpp:22-138): x is
    [B, D] or [B, D, T]; query_start_loc is refused with zeros(1) (:41-45);
    cache_seqlens / num_accepted_tokens are refused (:133-136).  Unlike the
    reference, ``activation`` is honoured (its binaries ignore it, :38).
    """
    import warnings
    if query_start_loc is not None:
        warnings.warn("npu_causal_conv1d_update does not support query_start_loc")
        return torch.zeros(1)
    if cache_seqlens is not None or num_accepted_tokens is not None:
        raise NotImplementedError("causal_conv1d_update does not support "
                                  "cache_seqlens or num_accepted_tokens")
    unsq = x.dim() == 2
    xs = x.unsqueeze(-1) if unsq else x
    B, D, T = xs.shape
    W = weight.size(1)
    S = conv_state.size(2)
    if weight.size(0) != D or conv_state.size(1) != D:
        raise ValueError("weight / conv_state dim mismatch")
    out = torch.empty_like(xs)
    idx = None
    if conv_state_indices is not None:
        idx = conv_state_indices.to(torch.int32).contiguous()
    w = weight if weight.dtype in (x.dtype, torch.float32) else weight.to(x.dtype)
    bvec = None
    if bias is not None:
        bvec = bias.to(w.dtype).contiguous()
    st = lib().xk_causal_conv1d_update(
        xs.data_ptr(), xs.stride(0), xs.stride(1), xs.stride(2),
        conv_state.data_ptr(), conv_state.stride(0), conv_state.stride(1),
        conv_state.stride(2), w.data_ptr(), w.stride(0), w.stride(1), _ptr(bvec),
        xk_dtype(w), _ptr(idx), int(pad_slot_id), conv_state.size(0),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), B, D, T, W, S,
        int(activation), xk_dtype(xs), _stream(x))
    check(st, "xk_causal_conv1d_update")
    return out.squeeze(-1) if unsq else out


def npu_causal_conv1d_update_v2(x: torch.Tensor, conv_state: torch.Tensor,
                                weight: torch.Tensor, activation: bool = True,
                                bias: Optional[torch.Tensor] = None,
                                conv_state_indices: Optional[torch.Tensor] = None,
                                query_start_loc: Optional[torch.Tensor] = None,
                                max_query_len: int = -1, pad_slot_id: int = -1,
                                block_idx_last_scheduled_token: Optional[torch.Tensor] = None,
                                initial_state_idx: Optional[torch.Tensor] = None,
                                validate_data: bool = False,
                                num_accepted_tokens: Optional[torch.Tensor] = None,
                                state_rule: int = 0):
    """Varlen causal conv1d with state slots (APC, spec decoding).

    Mirrors npu_causal_conv1d_update_v2
    (triton_npu/torch_api/npu_triton_causal_conv1d_update_v2.cpp:99-239) and
    its input preparation (:31-90): with query_start_loc x is [tokens, D];
    otherwise x is [B, D] or [B, D, T] and each batch row is one sequence.
    conv_state [lines, D, state_len] is read and written in place (no
    transposed copy).  ``state_rule`` 0 is the reference's final-state rule,
    1 keeps the last width-1 inputs of every sequence (full prefill).
    """
    if weight.dim() != 2:
        raise ValueError("causal_conv1d_update_v2 expects weight shape [dim, width].")
    if (block_idx_last_scheduled_token is None) != (initial_state_idx is None):
        raise ValueError("causal_conv1d_update_v2 expects both APC tensors or neither.")
    if conv_state.dim() != 3:
        raise ValueError("causal_conv1d_update_v2 expects conv_state shape "
                         "[num_cache_lines, dim, state_len].")
    dense = query_start_loc is None
    if dense:
        unsq = x.dim() == 2
        xw = x.unsqueeze(-1) if unsq else x
        B, D, T = xw.shape
        xt = xw.transpose(1, 2).contiguous().view(B * T, D)
        qsl = torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=x.device)
        mql = T
    else:
        if x.dim() != 2:
            raise ValueError("causal_conv1d_update_v2 expects x to be 2D "
                             "[num_tokens, dim] when query_start_loc is provided.")
        qsl = query_start_loc.to(torch.int32).contiguous()
        B = qsl.numel() - 1
        D = x.size(1)
        xt = x if x.stride(1) == 1 else x.contiguous()
        mql = max_query_len
        if mql < 0:
            mql = int((qsl[1:] - qsl[:-1]).max().item()) if B > 0 else 0
    W = weight.size(1)
    if not 1 <= W <= 6:
        raise ValueError(f"causal_conv1d_update_v2 expects width in [1, 6], got {W}")
    if weight.size(0) != D or conv_state.size(1) != D:
        raise ValueError("weight / conv_state dim mismatch")
    slots, s2d, sstride = None, 0, 0
    if conv_state_indices is not None:
        slots = conv_state_indices.to(torch.int32).contiguous()
        s2d = int(slots.dim() == 2)
        sstride = slots.stride(0) if s2d else 1
        if slots.size(0) != B:
            raise ValueError("conv_state_indices batch mismatch")
    last = init = acc = None
    if block_idx_last_scheduled_token is not None:
        last = block_idx_last_scheduled_token.to(torch.int32).contiguous()
        init = initial_state_idx.to(torch.int32).contiguous()
    if num_accepted_tokens is not None:
        acc = num_accepted_tokens.to(torch.int32).contiguous()
    # The kernel reads x in the state's dtype (reference :172) and the result
    # is returned in x's original dtype (:238).
    x_dtype = x.dtype
    if xt.dtype != conv_state.dtype:
        xt = xt.to(conv_state.dtype)
    w = weight if weight.dtype in (xt.dtype, torch.float32) else weight.to(xt.dtype)
    bvec = bias.to(w.dtype).contiguous() if bias is not None else None
    out = torch.empty_like(xt)
    st = lib().xk_causal_conv1d_varlen(
        xt.data_ptr(), xt.stride(0), xt.size(0), out.data_ptr(), out.stride(0),
        conv_state.data_ptr(), conv_state.stride(0), conv_state.stride(1),
        conv_state.stride(2), conv_state.size(0), conv_state.size(2),
        w.data_ptr(), w.stride(0), w.stride(1), _ptr(bvec), xk_dtype(w),
        qsl.data_ptr(), B, _ptr(slots), sstride, s2d, _ptr(init), _ptr(last),
        _ptr(acc), D, W, mql, int(state_rule), int(activation), int(pad_slot_id),
        xk_dtype(xt), _stream(x))
    check(st, "xk_causal_conv1d_varlen")
    out = out.to(x_dtype)
    if dense:
        o = out.view(B, T, D).transpose(1, 2)
        return o.squeeze(-1) if unsq else o.contiguous()
    return out


def npu_fused_recurrent_gated_delta_rule(
        q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
        beta: Optional[torch.Tensor] = None, scale: Optional[float] = None,
        initial_state: Optional[torch.Tensor] = None,
        inplace_final_state: bool = True,
        cu_seqlens: Optional[torch.Tensor] = None,
        ssm_state_indices: Optional[torch.Tensor] = None,
        num_accepted_tokens: Optional[torch.Tensor] = None,
        use_qk_l2norm_in_kernel: bool = True):
    """Recurrent gated delta rule; returns (o, final_state).

    Mirrors npu_fused_recurrent_gated_delta_rule
    (triton_npu/torch_api/npu_triton_recurrent_gated_delta_rule.cpp:54-247):
    q, k [B, T, H, K], v [B, T, HV, V], g / beta [B, T, HV]; B must be 1
    unless cu_seqlens is given; o is [B, T, HV, V] (squeezed NK dim);
    with inplace_final_state the returned state is initial_state itself.
    The reference binaries ignore use_qk_l2norm_in_kernel (always on); here
    it is honoured, with the compatibility default True.
    """
    B, T, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    if cu_seqlens is None and q.size(0) != 1:
        raise ValueError("batch size is not 1 when cu_seqlens is not provided")
    if initial_state is None:
        raise ValueError("initial_state must be provided")
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(K)
    N = cu_seqlens.numel() - 1 if cu_seqlens is not None else B
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    gc = g.contiguous()
    bc = beta.contiguous() if beta is not None else None
    o = torch.empty(B, T, HV, V, dtype=q.dtype, device=q.device)
    h0 = initial_state
    if h0.dtype != torch.float32 or not h0.is_contiguous():
        raise ValueError("initial_state must be contiguous float32")
    if inplace_final_state:
        final = h0
    else:
        final = torch.empty(N, HV, K, V, dtype=torch.float32, device=q.device)
    idx, s0, s1 = None, 0, 0
    if ssm_state_indices is not None:
        idx = ssm_state_indices.to(torch.int32).contiguous()
        s0 = idx.stride(0)
        s1 = idx.stride(1) if idx.dim() == 2 else 0
    acc = num_accepted_tokens.to(torch.int32).contiguous() if num_accepted_tokens is not None else None
    cu = cu_seqlens.contiguous() if cu_seqlens is not None else None
    st = lib().xk_gdn_recurrent(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), xk_dtype(qc), gc.data_ptr(),
        xk_dtype(gc), _ptr(bc), xk_dtype(bc) if bc is not None else 0, o.data_ptr(),
        h0.data_ptr(), h0.stride(0), final.data_ptr(), final.stride(0), h0.size(0),
        _ptr(cu), xk_dtype(cu) if cu is not None else 0, _ptr(idx), s0, s1,
        _ptr(acc), N, T if cu is None else 0, H, HV, K, V, sc,
        int(use_qk_l2norm_in_kernel), int(inplace_final_state), _stream(q))
    check(st, "xk_gdn_recurrent")
    return o, final


def npu_fused_gdn_gating(A_log: torch.Tensor, a: torch.Tensor, b: torch.Tensor,
                         dt_bias: torch.Tensor, beta: float = 1.0,
                         threshold: float = 20.0):
    """GDN gating; returns (g [1, batch, heads] fp32, beta_output [1, batch,
    heads] in b's dtype).

    Mirrors npu_fused_gdn_gating
    (triton_npu/torch_api/npu_triton_fused_gdn_gating.cpp:33-94):
    g = -exp(A_log) * softplus_{beta, threshold}(a + dt_bias),
    beta_output = sigmoid(b); A_log and dt_bias are fp32 [heads], a and b
    [batch, heads].
    """
    for t, name in ((A_log, "A_log"), (a, "a"), (b, "b"), (dt_bias, "dt_bias")):
        if not t.is_contiguous():
            raise ValueError(f"{name} tensor must be contiguous")
    if A_log.dtype != torch.float32:
        raise ValueError("A_log must be float32")
    if dt_bias.dtype != torch.float32:
        raise ValueError("dt_bias must be float32")
    if A_log.dim() != 1 or dt_bias.dim() != 1:
        raise ValueError("A_log and dt_bias must be 1D tensors")
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("a and b must be 2D tensors (batch, num_heads)")
    if b.dtype != a.dtype or b.shape != a.shape:
        raise ValueError("a and b must have the same dtype and shape")
    batch, heads = a.shape
    g = torch.empty(1, batch, heads, dtype=torch.float32, device=a.device)
    beta_out = torch.empty(1, batch, heads, dtype=b.dtype, device=b.device)
    st = lib().xk_fused_gdn_gating(A_log.data_ptr(), a.data_ptr(), b.data_ptr(),
                                   dt_bias.data_ptr(), g.data_ptr(), beta_out.data_ptr(),
                                   batch, heads, float(beta), float(threshold),
                                   xk_dtype(a), _stream(a))
    check(st, "xk_fused_gdn_gating")
    return g, beta_out


def npu_fused_sigmoid_gating_delta_rule_update(
        A_log: torch.Tensor, a: torch.Tensor, dt_bias: torch.Tensor, q: torch.Tensor,
        k: torch.Tensor, v: torch.Tensor, b: torch.Tensor,
        initial_state_source: torch.Tensor, initial_state_indices: torch.Tensor,
        cu_seqlens: torch.Tensor, scale: Optional[float] = None,
        use_qk_l2norm_in_kernel: bool = False, softplus_beta: float = 1.0,
        softplus_threshold: float = 20.0):
    """Recurrent gated delta rule with in-kernel gating; returns o [B, T,
    HV, V] and updates initial_state_source in place.

    Mirrors npu_fused_sigmoid_gating_delta_rule_update
    (triton_npu/torch_api/npu_triton_fused_sigmoid_gating_delta_rule_update.cpp:54-177):
    q, k [B, T, H, K], v [B, T, HV, V], a, b [B, T, HV], A_log, dt_bias fp32
    [HV], initial_state_source fp32 [slots, HV, K, V], initial_state_indices
    int32 [N], cu_seqlens int32 [N + 1].  A negative state index starts from
    zeros and leaves the pool untouched.
    """
    named = ((A_log, "A_log"), (a, "a"), (dt_bias, "dt_bias"), (q, "q"), (k, "k"),
             (v, "v"), (b, "b"), (initial_state_source, "initial_state_source"),
             (initial_state_indices, "initial_state_indices"), (cu_seqlens, "cu_seqlens"))
    for t, name in named:
        if not t.is_contiguous():
            raise ValueError(f"{name} tensor must be contiguous")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q/k must be 4D [B, T, H, K] and v 4D [B, T, HV, V]")
    B, T, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    N = cu_seqlens.numel() - 1
    if q.shape != k.shape:
        raise ValueError("q/k shape mismatch")
    if a.shape != (B, T, HV) or b.shape != a.shape:
        raise ValueError("a/b shape mismatch")
    if A_log.numel() != HV or dt_bias.numel() != HV:
        raise ValueError("A_log / dt_bias HV mismatch")
    if tuple(initial_state_source.shape[1:]) != (HV, K, V):
        raise ValueError("initial_state_source shape mismatch")
    if initial_state_indices.numel() != N:
        raise ValueError("initial_state_indices size must equal cu_seqlens size - 1")
    if HV % H != 0:
        raise ValueError("HV must be divisible by H")
    if A_log.dtype != torch.float32 or dt_bias.dtype != torch.float32:
        raise ValueError("A_log and dt_bias must be float32")
    if initial_state_source.dtype != torch.float32:
        raise ValueError("initial_state_source must be float32")
    if initial_state_indices.dtype != torch.int32 or cu_seqlens.dtype != torch.int32:
        raise ValueError("initial_state_indices and cu_seqlens must be int32")
    if b.dtype != a.dtype:
        raise ValueError("a and b must have the same dtype")
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(K)
    o = torch.empty(B, T, HV, V, dtype=q.dtype, device=q.device)
    st = lib().xk_gdn_sigmoid_gating_update(
        A_log.data_ptr(), a.data_ptr(), dt_bias.data_ptr(), float(softplus_beta),
        float(softplus_threshold), q.data_ptr(), k.data_ptr(), v.data_ptr(), b.data_ptr(),
        xk_dtype(a), o.data_ptr(), initial_state_source.data_ptr(),
        initial_state_source.stride(0), initial_state_source.size(0),
        initial_state_indices.data_ptr(), cu_seqlens.data_ptr(), N, H, HV, K, V, sc,
        int(use_qk_l2norm_in_kernel), xk_dtype(q), _stream(q))
    check(st, "xk_gdn_sigmoid_gating_update")
    return o


def npu_fused_qkvzba_split_reshape_cat(mixed_qkvz: torch.Tensor, mixed_ba: torch.Tensor,
                                       num_heads_qk: int, num_heads_v: int, head_qk: int,
                                       head_v: int):
    """Split of the GDN input projection; returns (mixed_qkv, z [rows,
    num_heads_v, head_v], b, a).

    Mirrors npu_fused_qkvzba_split_reshape_cat
    (triton_npu/torch_api/npu_triton_fused_qkvzba_split_reshape.cpp:116-230):
    rows of mixed_qkvz hold per-qk-head groups [q | k | v | z] and rows of
    mixed_ba groups [b | a]; v heads per qk head must be in [1, 4].
    """
    rph = num_heads_v // num_heads_qk
    if not (1 <= rph <= 4) or num_heads_v % num_heads_qk:
        raise ValueError(
            "npu_fused_qkvzba_split_reshape_cat only supports v_heads_per_qk in [1, 4], "
            f"but got {rph} for num_heads_qk={num_heads_qk} num_heads_v={num_heads_v}")
    rows = mixed_qkvz.size(0)
    qkv_dim = num_heads_qk * head_qk * 2 + num_heads_v * head_v
    q2 = mixed_qkvz.reshape(rows, -1)
    b2 = mixed_ba.reshape(rows, -1)
    if q2.stride(-1) != 1:
        q2 = q2.contiguous()
    if b2.stride(-1) != 1:
        b2 = b2.contiguous()
    mixed_qkv = torch.empty(rows, qkv_dim, dtype=mixed_qkvz.dtype, device=mixed_qkvz.device)
    z = torch.empty(rows, num_heads_v * head_v, dtype=mixed_qkvz.dtype, device=mixed_qkvz.device)
    b = torch.empty(rows, num_heads_v, dtype=mixed_ba.dtype, device=mixed_ba.device)
    a = torch.empty(rows, num_heads_v, dtype=mixed_ba.dtype, device=mixed_ba.device)
    st = lib().xk_fused_qkvzba_split_reshape_cat(
        q2.data_ptr(), q2.stride(0), b2.data_ptr(), b2.stride(0), mixed_qkv.data_ptr(),
        z.data_ptr(), b.data_ptr(), a.data_ptr(), rows, num_heads_qk, num_heads_v, head_qk,
        head_v, xk_dtype(q2), xk_dtype(b2), _stream(mixed_qkvz))
    check(st, "xk_fused_qkvzba_split_reshape_cat")
    return mixed_qkv, z.view(rows, num_heads_v, head_v), b, a


def npu_chunk_gated_delta_rule(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               g: torch.Tensor, beta: torch.Tensor,
                               scale: Optional[float] = None,
                               initial_state: Optional[torch.Tensor] = None,
                               output_final_state: bool = False,
                               cu_seqlens: Optional[torch.Tensor] = None,
                               head_first: bool = False,
                               use_qk_l2norm_in_kernel: bool = False):
    """Chunked gated delta rule (chunk 64); returns (o, final_state or None).

    Mirrors npu_chunk_gated_delta_rule
    (triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:556-642):
    q, k [B, T, H, K], v [B, T, HV, V] bf16, g / beta [B, T, HV];
    head_first must be False; initial_state [N, HV, K, V] (bf16 or fp32)
    is read in fp32; the final state is fp32.  Without cu_seqlens the B
    rows are B sequences of T tokens.  The whole pipeline runs on the
    device with no host synchronisation.
    """
    if head_first:
        raise ValueError("chunk_gated_delta_rule only supports head_first=false.")
    if not (q.dtype == k.dtype == v.dtype == torch.bfloat16):
        raise ValueError("chunk_gated_delta_rule expects q/k/v to be bfloat16.")
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    if q.shape != k.shape:
        raise ValueError("q and k must have the same shape.")
    if HV % H:
        raise ValueError("num_heads_v must be divisible by num_heads_qk")
    if beta.shape != (B, T, HV) or g.shape != (B, T, HV):
        raise ValueError("beta / g must have shape [B, T, H].")
    dev = q.device
    if cu_seqlens is None:
        cu = torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=dev)
    else:
        cu = cu_seqlens.contiguous()
        if cu.dtype not in (torch.int32, torch.int64):
            cu = cu.to(torch.int32)
    N = cu.numel() - 1
    total = B * T
    sc = float(scale) if scale is not None else K ** -0.5
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    gc, bc = g.contiguous(), beta.contiguous()
    h0 = None
    if initial_state is not None:
        h0 = initial_state.to(torch.float32).contiguous()
    fin = torch.empty(N, HV, K, V, dtype=torch.float32, device=dev) if output_final_state else None
    o = torch.empty(B, T, HV, V, dtype=q.dtype, device=dev)
    ws_bytes = lib().xk_gdn_chunk_workspace_bytes(total, N, HV)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    st = lib().xk_gdn_chunk_fwd(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), xk_dtype(qc), gc.data_ptr(),
        xk_dtype(gc), bc.data_ptr(), xk_dtype(bc), o.data_ptr(), _ptr(h0), _ptr(fin),
        cu.data_ptr(), xk_dtype(cu), N, total, H, HV, K, V, sc,
        int(use_qk_l2norm_in_kernel), ws.data_ptr(), ws.numel(), _stream(q))
    check(st, "xk_gdn_chunk_fwd")
    return o, fin


# ---------------------------------------------------------------------------
# The chunked pipeline stage by stage
# ---------------------------------------------------------------------------
def _seqs(B: int, T: int, cu_seqlens: Optional[torch.Tensor], dev):
    """(cu tensor on dev, N): the reference's varlen table, or B sequences
    of T tokens when cu_seqlens is None (chunk.py's batch convention)."""
    if cu_seqlens is None:
        return torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=dev), B
    cu = cu_seqlens.to(dev).contiguous()
    if cu.dtype not in (torch.int32, torch.int64):
        cu = cu.to(torch.int32)
    return cu, cu.numel() - 1


def _num_chunks(cu: torch.Tensor, total: int, chunk: int = 64) -> int:
    """Chunks of all sequences, with the kernels' clamping of cu_seqlens to
    [0, total] (the reference's infer_total_chunks, also a host read of
    cu_seqlens: npu_triton_chunk_gated_delta_rule.cpp:116-138)."""
    c = cu.detach().to("cpu", torch.int64).clamp(0, total)
    lens = (c[1:] - c[:-1]).clamp(min=0)
    return int(((lens + chunk - 1) // chunk).sum())


def _stage_ws(N: int, dev) -> torch.Tensor:
    return torch.empty(max(lib().xk_gdn_stage_workspace_bytes(N), 1),
                       dtype=torch.uint8, device=dev)


def npu_chunk_local_cumsum(g: torch.Tensor, chunk_size: int,
                           cu_seqlens: Optional[torch.Tensor] = None):
    """Per-chunk inclusive cumsum of g [B, T, H] along T; fp32 out.

    Mirrors npu_chunk_local_cumsum
    (triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:151-227);
    its H <= 64 launch limit (:173-176) does not apply here.
    """
    if g.dim() != 3:
        raise ValueError("chunk_local_cumsum expects g to have shape [B, T, H].")
    if chunk_size <= 0 or chunk_size & (chunk_size - 1):
        raise ValueError("chunk_local_cumsum expects chunk_size to be a power of two")
    B, T, H = g.shape
    cu, N = _seqs(B, T, cu_seqlens, g.device)
    gc = g.contiguous()
    out = torch.empty(g.shape, dtype=torch.float32, device=g.device)
    st = lib().xk_chunk_local_cumsum(gc.data_ptr(), xk_dtype(gc), out.data_ptr(), B * T, H,
                                     cu.data_ptr(), xk_dtype(cu), N, chunk_size, _stream(g))
    check(st, "xk_chunk_local_cumsum")
    return out


def npu_chunk_scaled_dot_kkt_fwd(k: torch.Tensor, beta: torch.Tensor,
                                 g_cumsum: Optional[torch.Tensor], chunk_size: int = 64,
                                 cu_seqlens: Optional[torch.Tensor] = None):
    """A [B, T, H, 64] fp32 = strict_tril(beta_i (k_i . k_j) exp(gc_i - gc_j)).

    Mirrors npu_chunk_scaled_dot_kkt_fwd
    (triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:229-297).
    """
    if chunk_size != 64:
        raise ValueError("chunk_scaled_dot_kkt_fwd supports chunk_size=64")
    B, T, Hg, K = k.shape
    H = beta.size(2)
    cu, N = _seqs(B, T, cu_seqlens, k.device)
    kc, bc = k.contiguous(), beta.contiguous()
    gcum = g_cumsum.to(torch.float32).contiguous() if g_cumsum is not None else None
    A = torch.empty(B, T, H, 64, dtype=torch.float32, device=k.device)
    ws = _stage_ws(N, k.device)
    st = lib().xk_chunk_scaled_dot_kkt(
        kc.data_ptr(), xk_dtype(kc), bc.data_ptr(), xk_dtype(bc), _ptr(gcum), A.data_ptr(),
        B * T, Hg, H, K, cu.data_ptr(), xk_dtype(cu), N, ws.data_ptr(), ws.numel(), _stream(k))
    check(st, "xk_chunk_scaled_dot_kkt")
    return A


def npu_solve_tril(A: torch.Tensor, chunk_size: int = 64,
                   cu_seqlens: Optional[torch.Tensor] = None,
                   output_dtype: torch.dtype = torch.float32):
    """Ai = (I + A)^-1 per chunk, [B, T, H, 64] in output_dtype.

    Mirrors npu_solve_tril
    (triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:299-395).
    """
    if chunk_size != 64:
        raise ValueError("chunk_gated_delta_rule solve_tril wrapper only supports chunk_size=64.")
    B, T, H, C = A.shape
    if C != 64:
        raise ValueError("solve_tril expects A of shape [B, T, H, 64]")
    cu, N = _seqs(B, T, cu_seqlens, A.device)
    Ac = A.to(torch.float32).contiguous()
    Ai = torch.empty(A.shape, dtype=output_dtype, device=A.device)
    ws = _stage_ws(N, A.device)
    st = lib().xk_solve_tril(Ac.data_ptr(), Ai.data_ptr(), xk_dtype(Ai), B * T, H,
                             cu.data_ptr(), xk_dtype(cu), N, ws.data_ptr(), ws.numel(), _stream(A))
    check(st, "xk_solve_tril")
    return Ai


def npu_recompute_w_u_fwd(k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                          g_cumsum: torch.Tensor, A: torch.Tensor,
                          cu_seqlens: Optional[torch.Tensor] = None):
    """(w, u) = (Ai (k beta exp(gc)), Ai (v beta)), w like k, u like v.

    Mirrors npu_recompute_w_u_fwd
    (triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:397-475).
    """
    B, T, Hg, K = k.shape
    H, V = v.size(2), v.size(3)
    cu, N = _seqs(B, T, cu_seqlens, k.device)
    kc, vc, bc = k.contiguous(), v.contiguous(), beta.contiguous()
    gcum = g_cumsum.to(torch.float32).contiguous()
    Ac = A.contiguous()
    w = torch.empty(B, T, H, K, dtype=k.dtype, device=k.device)
    u = torch.empty_like(vc)
    ws = _stage_ws(N, k.device)
    st = lib().xk_recompute_w_u(
        kc.data_ptr(), vc.data_ptr(), xk_dtype(kc), bc.data_ptr(), xk_dtype(bc),
        gcum.data_ptr(), Ac.data_ptr(), xk_dtype(Ac), w.data_ptr(), u.data_ptr(), B * T, Hg, H,
        K, V, cu.data_ptr(), xk_dtype(cu), N, ws.data_ptr(), ws.numel(), _stream(k))
    check(st, "xk_recompute_w_u")
    return w, u


def npu_chunk_gated_delta_rule_fwd_h(k: torch.Tensor, w: torch.Tensor, u: torch.Tensor,
                                     g: Optional[torch.Tensor] = None,
                                     initial_state: Optional[torch.Tensor] = None,
                                     output_final_state: bool = False,
                                     chunk_size: int = 64, save_new_value: bool = True,
                                     cu_seqlens: Optional[torch.Tensor] = None,
                                     chunk_offsets: Optional[torch.Tensor] = None):
    """Returns (h [B, NT, H, K, V] k-dtype, v_new or None, final_state or None).

    Mirrors npu_chunk_gated_delta_rule_fwd_h
    (triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:644-802):
    g is the per-chunk cumsum of the log-decay; h[c] is the state entering
    chunk c.  chunk_offsets, if given, must match cu_seqlens (the chunk
    offsets are recomputed on the device).
    """
    if chunk_size != 64:
        raise ValueError("chunk_gated_delta_rule_fwd_h only supports chunk_size=64")
    for name, t in (("k", k), ("w", w), ("u", u)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"chunk_gated_delta_rule_fwd_h expects {name} to be bfloat16")
    B, T, Hg, K = k.shape
    H, V = u.size(2), u.size(3)
    cu, N = _seqs(B, T, cu_seqlens, k.device)
    NT = _num_chunks(cu, B * T)
    if chunk_offsets is not None and chunk_offsets.numel() != N + 1:
        raise ValueError("chunk_offsets must have N + 1 entries")
    kc, wc, uc = k.contiguous(), w.contiguous(), u.contiguous()
    gcum = g.to(torch.float32).contiguous() if g is not None else None
    h0 = initial_state.to(torch.float32).contiguous() if initial_state is not None else None
    h = torch.empty(B if cu_seqlens is None else 1, NT // (B if cu_seqlens is None else 1),
                    H, K, V, dtype=k.dtype, device=k.device)
    v_new = torch.empty_like(uc) if save_new_value else None
    fin = torch.empty(N, H, K, V, dtype=torch.float32, device=k.device) if output_final_state else None
    ws = _stage_ws(N, k.device)
    st = lib().xk_chunk_fwd_h(
        kc.data_ptr(), wc.data_ptr(), uc.data_ptr(), xk_dtype(kc), _ptr(gcum), _ptr(h0),
        h.data_ptr(), NT, _ptr(v_new), _ptr(fin), B * T, Hg, H, K, V, cu.data_ptr(),
        xk_dtype(cu), N, ws.data_ptr(), ws.numel(), _stream(k))
    check(st, "xk_chunk_fwd_h")
    return h, v_new, fin


def npu_chunk_fwd_o(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, h: torch.Tensor,
                    g_cumsum: Optional[torch.Tensor], scale: float, chunk_size: int = 64,
                    cu_seqlens: Optional[torch.Tensor] = None):
    """o = scale (exp(gc) (q h_c) + tril(q k^T exp(gc_i - gc_j)) v), like v.

    Mirrors npu_chunk_fwd_o
    (triton_npu/torch_api/npu_triton_chunk_gated_delta_rule.cpp:477-554).
    """
    if chunk_size != 64:
        raise ValueError("chunk_fwd_o supports chunk_size=64")
    B, T, Hg, K = q.shape
    H, V = v.size(2), v.size(3)
    cu, N = _seqs(B, T, cu_seqlens, q.device)
    qc, kc, vc, hc = q.contiguous(), k.contiguous(), v.contiguous(), h.contiguous()
    NT = hc.numel() // (H * K * V)
    gcum = g_cumsum.to(torch.float32).contiguous() if g_cumsum is not None else None
    o = torch.empty_like(vc)
    ws = _stage_ws(N, q.device)
    st = lib().xk_chunk_fwd_o(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), hc.data_ptr(), NT, xk_dtype(qc),
        _ptr(gcum), o.data_ptr(), float(scale), B * T, Hg, H, K, V, cu.data_ptr(),
        xk_dtype(cu), N, ws.data_ptr(), ws.numel(), _stream(q))
    check(st, "xk_chunk_fwd_o")
    return o


def _check_conv_decode(mixed_qkv, conv_state, conv_weight, ssm_state, num_heads_qk,
                       num_heads_v, head_k, head_v):
    if mixed_qkv.dim() != 2:
        raise ValueError("gdn_conv_decode expects mixed_qkv [B, D]")
    B, D = mixed_qkv.shape
    if D != 2 * num_heads_qk * head_k + num_heads_v * head_v:
        raise ValueError("mixed_qkv width does not match the head layout")
    # The kernel indexes ssm_state as dense fp32 [slots, HV, K, V] (slot
    # stride from stride(0)) and conv_state in mixed_qkv's dtype.
    if ssm_state.dtype != torch.float32:
        raise ValueError("ssm_state must be float32")
    if (ssm_state.dim() != 4
            or tuple(ssm_state.shape[1:]) != (num_heads_v, head_k, head_v)):
        raise ValueError("ssm_state must have shape [slots, num_heads_v, head_k, head_v]")
    if ssm_state.stride()[1:] != (head_k * head_v, head_v, 1):
        raise ValueError("ssm_state must be contiguous within each slot")
    if conv_state.dtype != mixed_qkv.dtype:
        raise ValueError("conv_state must have mixed_qkv's dtype")
    if conv_state.dim() != 3 or conv_state.size(1) != D:
        raise ValueError("conv_state must have shape [lines, D, state_len]")
    if conv_weight.dim() != 2 or conv_weight.size(0) != D:
        raise ValueError("conv_weight must have shape [D, width]")
    return B, D


def _conv_decode_common(mixed_qkv, conv_state, conv_weight, ssm_state, conv_bias,
                        conv_state_indices, ssm_state_indices, pad_slot_id, head_k):
    """Leading C-ABI arguments shared by both fused decode entry points."""
    x = mixed_qkv if mixed_qkv.stride(1) == 1 else mixed_qkv.contiguous()
    w = conv_weight
    cb = conv_bias.to(w.dtype).contiguous() if conv_bias is not None else None
    ci = conv_state_indices.to(torch.int32).contiguous() if conv_state_indices is not None else None
    si = ssm_state_indices.to(torch.int32).contiguous() if ssm_state_indices is not None else None
    head = (x.data_ptr(), x.stride(0), conv_state.data_ptr(), conv_state.stride(0),
            conv_state.stride(1), conv_state.stride(2), conv_state.size(0),
            conv_state.size(2), w.data_ptr(), w.stride(0), w.stride(1), _ptr(cb),
            xk_dtype(w), w.size(1), _ptr(ci), int(pad_slot_id))
    keep = (x, cb, ci, si)  # alive until the launch is enqueued
    return x, head, si, keep


def gdn_conv_decode(mixed_qkv: torch.Tensor, conv_state: torch.Tensor,
                    conv_weight: torch.Tensor, g: torch.Tensor,
                    beta: Optional[torch.Tensor], ssm_state: torch.Tensor,
                    num_heads_qk: int, num_heads_v: int, head_k: int = 128,
                    head_v: int = 128, scale: Optional[float] = None,
                    conv_bias: Optional[torch.Tensor] = None,
                    conv_state_indices: Optional[torch.Tensor] = None,
                    ssm_state_indices: Optional[torch.Tensor] = None,
                    pad_slot_id: int = -1, use_qk_l2norm: bool = True):
    """One fused decode step: conv1d update + SiLU of mixed_qkv [B, D],
    split into q / k / v heads, l2norm, one gated-delta-rule step on
    ssm_state (updated in place).  Returns o [B, HV, V]."""
    B, D = _check_conv_decode(mixed_qkv, conv_state, conv_weight, ssm_state, num_heads_qk,
                              num_heads_v, head_k, head_v)
    if tuple(g.shape) != (B, num_heads_v):
        raise ValueError("g must have shape [B, num_heads_v]")
    if beta is not None and tuple(beta.shape) != (B, num_heads_v):
        raise ValueError("beta must have shape [B, num_heads_v]")
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(head_k)
    x, head, si, _keep = _conv_decode_common(mixed_qkv, conv_state, conv_weight, ssm_state,
                                              conv_bias, conv_state_indices,
                                              ssm_state_indices, pad_slot_id, head_k)
    gc = g.contiguous()
    bc = beta.contiguous() if beta is not None else None
    o = torch.empty(B, num_heads_v, head_v, dtype=x.dtype, device=x.device)
    st = lib().xk_gdn_conv_decode(
        *head, gc.data_ptr(), xk_dtype(gc), _ptr(bc), xk_dtype(bc) if bc is not None else 0,
        ssm_state.data_ptr(), ssm_state.stride(0), ssm_state.size(0), _ptr(si),
        o.data_ptr(), B, num_heads_qk, num_heads_v, head_k, head_v, sc,
        int(use_qk_l2norm), xk_dtype(x), _stream(x))
    check(st, "xk_gdn_conv_decode")
    return o


def gdn_conv_gating_decode(mixed_qkv: torch.Tensor, conv_state: torch.Tensor,
                           conv_weight: torch.Tensor, A_log: torch.Tensor, a: torch.Tensor,
                           dt_bias: torch.Tensor, b: torch.Tensor, ssm_state: torch.Tensor,
                           num_heads_qk: int, num_heads_v: int, head_k: int = 128,
                           head_v: int = 128, scale: Optional[float] = None,
                           conv_bias: Optional[torch.Tensor] = None,
                           conv_state_indices: Optional[torch.Tensor] = None,
                           ssm_state_indices: Optional[torch.Tensor] = None,
                           pad_slot_id: int = -1, softplus_beta: float = 1.0,
                           softplus_threshold: float = 20.0, use_qk_l2norm: bool = True):
    """gdn_conv_decode with the gating in the kernel: g = -exp(A_log) *
    softplus(a + dt_bias) and beta = sigmoid(b) per (row, v head), in fp32
    (as npu_fused_sigmoid_gating_delta_rule_update forms them).  a, b
    [B, HV]; A_log, dt_bias fp32 [HV].  Returns o [B, HV, V]."""
    B, D = _check_conv_decode(mixed_qkv, conv_state, conv_weight, ssm_state, num_heads_qk,
                              num_heads_v, head_k, head_v)
    for t, name in ((a, "a"), (b, "b")):
        if tuple(t.shape) != (B, num_heads_v):
            raise ValueError(f"{name} must have shape [B, num_heads_v]")
    if a.dtype != b.dtype:
        raise ValueError("a and b must have the same dtype")
    for t, name in ((A_log, "A_log"), (dt_bias, "dt_bias")):
        if t.dtype != torch.float32 or t.numel() != num_heads_v:
            raise ValueError(f"{name} must be float32 [num_heads_v]")
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(head_k)
    x, head, si, _keep = _conv_decode_common(mixed_qkv, conv_state, conv_weight, ssm_state,
                                              conv_bias, conv_state_indices,
                                              ssm_state_indices, pad_slot_id, head_k)
    ac, bc = a.contiguous(), b.contiguous()
    al, db = A_log.contiguous(), dt_bias.contiguous()
    o = torch.empty(B, num_heads_v, head_v, dtype=x.dtype, device=x.device)
    st = lib().xk_gdn_conv_gating_decode(
        *head, al.data_ptr(), ac.data_ptr(), db.data_ptr(), bc.data_ptr(), xk_dtype(ac),
        float(softplus_beta), float(softplus_threshold), ssm_state.data_ptr(),
        ssm_state.stride(0), ssm_state.size(0), _ptr(si), o.data_ptr(), B, num_heads_qk,
        num_heads_v, head_k, head_v, sc, int(use_qk_l2norm), xk_dtype(x), _stream(x))
    check(st, "xk_gdn_conv_gating_decode")
    return o


def npu_l2norm_last_dim(x: torch.Tensor, eps: float = 1e-6,
                        output_dtype: Optional[torch.dtype] = None):
    """x * rsqrt(sum(x^2) + eps) over the last dim.

    Mirrors npu_l2norm_last_dim (triton_npu/torch_api/npu_triton_l2norm.cpp:
    60-109), which accepts bf16 only and returns x's dtype; this accepts
    f32/bf16/f16 and an optional output dtype.
    """
    if x.dim() < 1 or x.size(-1) == 0:
        raise ValueError("npu_l2norm_last_dim expects hidden dim > 0")
    xc = x.contiguous()
    y = torch.empty(x.shape, dtype=output_dtype or x.dtype, device=x.device)
    rows = xc.numel() // x.size(-1)
    st = lib().xk_l2norm_last_dim(xc.data_ptr(), y.data_ptr(), rows,
                                  x.size(-1), float(eps), xk_dtype(xc),
                                  xk_dtype(y), _stream(x))
    check(st, "xk_l2norm_last_dim")
    return y
