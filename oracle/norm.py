"""CPU restatements of the normalisation references (test infrastructure).

layer_norm_fwd: triton_npu/test/triton_layernorm_fwd_test.cpp:37-116
  (layer_norm_golden_cpu) and triton_npu/triton_src/test_layernorm_fwd.py:
  1529-1565 (_golden_ref).  The statistics (mean, rstd) that the golden does
  not return follow the kernel definition test_layernorm_fwd.py:1166-1178:
  mean = sum(x)/G, var = sum((x-mean)^2)/G, rstd = 1/sqrt(var+eps), stored
  at group*M + row.
gemma_rms_norm: no reference implementation exists (closed CANN builtin
  aclnnGemmaRmsNorm, ascendc_npu/gemma_rms_norm.cpp:54); restated as the
  Gemma form x * rsqrt(mean(x^2)+eps) * (1+gamma) in fp32.  Pinned by its
  reduction to RMSNorm with weight (1+gamma) (torch.nn.functional.rms_norm).
l2norm_last_dim: triton_npu/triton_src/test_l2norm.py:91-94 (l2norm_ref).

Pins (tests/test_oracle_norm.py): torch.layer_norm / F.rms_norm library
routines, a float64 numpy per-(row, group) loop for the stats layout,
normalised-output moments, and F.normalize for the L2 norm.
"""
from __future__ import annotations

from typing import Optional

import torch


def _gate(z: torch.Tensor) -> torch.Tensor:
    return z * torch.sigmoid(z)


def layer_norm_fwd(x: torch.Tensor, weight: torch.Tensor,
                   bias: Optional[torch.Tensor], eps: float,
                   z: Optional[torch.Tensor] = None, group_size: int = -1,
                   norm_before_gate: bool = True, is_rms_norm: bool = False,
                   dtype: torch.dtype = torch.float32):
    """Returns (y, mean, rstd) in `dtype`; mean is None for RMS norm.

    Follows layer_norm_golden_cpu (triton_layernorm_fwd_test.cpp:37-116):
    gate before the statistics when z is given and not norm_before_gate, a
    per-group normalisation, then y * weight (+ bias), then the gate after.
    """
    N = x.shape[-1]
    G = group_size if group_size > 0 else N
    xs = x.reshape(-1, N).to(dtype)
    M = xs.shape[0]
    ng = N // G
    zs = z.reshape(-1, N).to(dtype) if z is not None else None
    if zs is not None and not norm_before_gate:
        xs = xs * _gate(zs)
    xg = xs.reshape(M, ng, G)
    if is_rms_norm:
        var = (xg * xg).mean(-1, keepdim=True)
        mean = None
        xhat = xg * (1.0 / torch.sqrt(var + eps))
    else:
        mu = xg.mean(-1, keepdim=True)
        var = ((xg - mu) ** 2).mean(-1, keepdim=True)
        xhat = (xg - mu) * (1.0 / torch.sqrt(var + eps))
        mean = mu.reshape(M, ng).t().reshape(-1)
    rstd = (1.0 / torch.sqrt(var + eps)).reshape(M, ng).t().reshape(-1)
    y = xhat.reshape(M, N) * weight.to(dtype)
    if bias is not None:
        y = y + bias.to(dtype)
    if zs is not None and norm_before_gate:
        y = y * _gate(zs)
    return y.reshape(x.shape), mean, rstd


def gemma_rms_norm(x: torch.Tensor, gamma: torch.Tensor, eps: float,
                   dtype: torch.dtype = torch.float32):
    """Returns (y, rstd[M]) with y = x * rsqrt(mean(x^2)+eps) * (1+gamma)."""
    N = gamma.numel()
    xs = x.reshape(-1, N).to(dtype)
    var = (xs * xs).mean(-1, keepdim=True)
    rstd = 1.0 / torch.sqrt(var + eps)
    y = xs * rstd * (1.0 + gamma.reshape(-1).to(dtype))
    return y.reshape(x.shape), rstd.reshape(-1)


def l2norm_last_dim(x: torch.Tensor, eps: float = 1e-6,
                    dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """x * rsqrt(sum(x^2) + eps) (test_l2norm.py:91-94), kept in `dtype`."""
    xf = x.to(dtype)
    return xf * torch.rsqrt((xf * xf).sum(-1, keepdim=True) + eps)
