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
# a2 / a3 / a6a: normalisation
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
