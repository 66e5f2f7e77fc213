"""CPU restatement of split_rmsnorm_rope (test infrastructure).

Follows the CPU golden triton_npu/test/triton_split_rmsnorm_rope_test.cpp:
88-136 (RmsNorm, RotateHalf, ApplyRope, Ref) and the Python reference
triton_npu/triton_src/test_split_rmsnorm_rope.py:277-356 (custom_rope,
split_rmsnorm_rope_ref, rms_norm): q and k heads are RMS-normalised with
1/sqrt(mean(x^2)+eps) * w (+ b), then rotated as x*cos + rotate_half(x)*sin
with rotate_half(x) = cat(-x2, x1); v passes through.

neox_cos_sin builds the per-token cos/sin rows the way the reference's ATB
rope consumes a neox cos_sin_cache (ops_npu/rope_atb.cpp:16-23):
freqs = pos * inv_freq, cos = cat(cos f, cos f), sin = cat(sin f, sin f).

rope_inplace_ref restates rope_ref of triton_npu/triton_src/
test_rope_inplace.py:66-94: GPT-J (interleaved) rotation of the last
rope_dim elements, out = x*cos + rotate(x)*sin with rotate(x)[2i] = -x[2i+1]
and rotate(x)[2i+1] = x[2i], rounded to x's dtype.

Pins (tests/test_oracle_rope.py): F.rms_norm for the norm, a complex-number
rotation (x1 + i x2)(cos + i sin) for the rotate-half sign convention and
(x[2i] + i x[2i+1])(cos + i sin) for the interleaved one, pair-norm
preservation, and position 0 (cos 1, sin 0) reducing to the identity.
"""
from __future__ import annotations

from typing import Optional

import torch


def inv_freq_table(head_dim: int, theta: float) -> torch.Tensor:
    """fp32 inverse frequencies theta^(-2i/head_dim), i < head_dim/2."""
    i = torch.arange(0, head_dim, 2, dtype=torch.float64)
    return (1.0 / (theta ** (i / head_dim))).to(torch.float32)


def neox_cos_sin(positions: torch.Tensor, inv_freq: torch.Tensor):
    """cos/sin rows [T, head_dim] in fp32 (freqs computed in fp32)."""
    f = positions.to(torch.float32)[:, None] * inv_freq[None, :]
    c, s = torch.cos(f), torch.sin(f)
    return torch.cat([c, c], -1), torch.cat([s, s], -1)


def _rms(x, w, eps, b=None, dtype=torch.float32):
    xf = x.to(dtype)
    out = xf * (1.0 / torch.sqrt((xf * xf).mean(-1, keepdim=True) + eps)) * w.to(dtype)
    if b is not None:
        out = out + b.to(dtype)
    return out


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], -1)


def split_rmsnorm_rope(qkv: torch.Tensor, sin: torch.Tensor, cos: torch.Tensor,
                       q_weight: torch.Tensor, k_weight: torch.Tensor,
                       q_hidden: int, kv_hidden: int, head_dim: int, eps: float,
                       q_bias: Optional[torch.Tensor] = None,
                       k_bias: Optional[torch.Tensor] = None,
                       dtype: torch.dtype = torch.float32):
    """Returns (q [T, q_hidden], k [T, kv_hidden], v [T, kv_hidden]) in dtype."""
    T = qkv.shape[0]
    q = qkv[:, :q_hidden].reshape(T, -1, head_dim)
    k = qkv[:, q_hidden:q_hidden + kv_hidden].reshape(T, -1, head_dim)
    v = qkv[:, q_hidden + kv_hidden:q_hidden + 2 * kv_hidden]
    qn = _rms(q, q_weight, eps, q_bias, dtype)
    kn = _rms(k, k_weight, eps, k_bias, dtype)
    c = cos.to(dtype)[:, None, :]
    s = sin.to(dtype)[:, None, :]
    qo = qn * c + _rotate_half(qn) * s
    ko = kn * c + _rotate_half(kn) * s
    return qo.reshape(T, q_hidden), ko.reshape(T, kv_hidden), v.to(dtype)


def rope_inplace_ref(x: torch.Tensor, sin: torch.Tensor, cos: torch.Tensor,
                     rope_dim: int) -> torch.Tensor:
    """x [bsz, hidden] or [bsz, heads, hidden]; sin / cos [bsz, rope_dim].
    Returns the rotated copy of x (same dtype; the prefix is unchanged)."""
    orig = x.dtype
    pre = x[..., :-rope_dim] if rope_dim < x.shape[-1] else None
    xr = x[..., -rope_dim:].float()
    s, c = sin.float(), cos.float()
    if x.dim() == 3:
        s, c = s.unsqueeze(1), c.unsqueeze(1)
    rot = torch.empty_like(xr)
    rot[..., ::2] = -xr[..., 1::2]
    rot[..., 1::2] = xr[..., ::2]
    out = (xr * c + rot * s).to(orig)
    return torch.cat([pre, out], dim=-1) if pre is not None else out
