"""CPU restatements of the GDN gating references (test infrastructure).

fused_gdn_gating: torch_fused_gdn_gating of
  triton_npu/triton_src/test_fused_gdn_gating.py:45-57 and of
  triton_npu/test/triton_fused_gdn_gating_test.cpp (torch_fused_gdn_gating):
  g = -exp(A_log) * softplus_{beta, threshold}(a + dt_bias) in fp32, and
  beta_out = sigmoid(b) in b's dtype.
sigmoid_gating_delta_rule_update: torch_sigmoid_gating_delta_rule_update of
  triton_npu/triton_src/test_fused_sigmoid_gating_delta_rule_update.py:178-222,
  a per-sequence, per-token loop over the state pool with the gating
  computed from a and b.  By default it follows the kernel's arithmetic
  (py:79-104): beta = sigmoid(b) and q/k normalised by 1/sqrt(sum^2 + 1e-6)
  in fp32, neither rounded.  ref_rounding=True reproduces the CPU ref
  instead, which normalises with F.normalize and rounds q/k to their input
  dtype (py:197-198) and evaluates b.sigmoid() in b's dtype (py:202).

Pins (tests/test_oracle_gating.py): softplus against
torch.nn.functional.softplus and pure-Python math values (ln 2 at zero, the
threshold branch, beta scaling), sigmoid symmetry, and the update against
oracle.gdn.recurrent_gdn (itself pinned by known answers) fed with the
gating of fused_gdn_gating, including negative state indices.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def softplus(x: torch.Tensor, beta: float = 1.0, threshold: float = 20.0) -> torch.Tensor:
    """log(1 + exp(beta x)) / beta where beta x <= threshold, else x
    (test_fused_gdn_gating.py:33-35)."""
    bx = beta * x
    return torch.where(bx <= threshold, torch.log1p(torch.exp(bx)) / beta, x)


def gating(A_log, a, b, dt_bias, beta: float = 1.0, threshold: float = 20.0,
           dtype=torch.float32):
    """(g, sigmoid(b)) in `dtype` for a, b [..., heads] and A_log, dt_bias
    [heads]; neither output is rounded."""
    x = a.to(dtype) + dt_bias.to(dtype)
    g = -torch.exp(A_log.to(dtype)) * softplus(x, beta, threshold)
    return g, torch.sigmoid(b.to(dtype))


def fused_gdn_gating(A_log, a, b, dt_bias, beta: float = 1.0, threshold: float = 20.0):
    """a, b [batch, heads] -> (g [1, batch, heads] fp32, beta_out [1, batch,
    heads] in b's dtype), as npu_fused_gdn_gating returns them."""
    g, s = gating(A_log, a, b, dt_bias, beta, threshold, torch.float32)
    return g.unsqueeze(0), s.to(b.dtype).unsqueeze(0)


def sigmoid_gating_delta_rule_update(A_log, a, dt_bias, q, k, v, b, initial_state,
                                     state_indices, cu_seqlens, scale: float,
                                     use_qk_l2norm: bool, softplus_beta: float = 1.0,
                                     softplus_threshold: float = 20.0,
                                     ref_rounding: bool = False, dtype=torch.float64):
    """q, k [B, T, H, K]; v [B, T, HV, V]; a, b [B, T, HV]; initial_state
    [slots, HV, K, V] (not modified); state_indices [N]; cu_seqlens [N + 1]
    over the B*T token rows.  Returns (o [B, T, HV, V] in `dtype`, new state
    pool)."""
    B, T, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    rep = HV // H
    q2 = q.reshape(B * T, H, K).repeat_interleave(rep, 1)
    k2 = k.reshape(B * T, H, K).repeat_interleave(rep, 1)
    if use_qk_l2norm:
        if ref_rounding:
            q2 = F.normalize(q2.float(), p=2, dim=-1, eps=1e-6).to(q.dtype)
            k2 = F.normalize(k2.float(), p=2, dim=-1, eps=1e-6).to(k.dtype)
            qf, kf = q2.to(dtype), k2.to(dtype)
        else:
            qf, kf = q2.to(dtype), k2.to(dtype)
            qf = qf / torch.sqrt((qf * qf).sum(-1, keepdim=True) + 1e-6)
            kf = kf / torch.sqrt((kf * kf).sum(-1, keepdim=True) + 1e-6)
    else:
        qf, kf = q2.to(dtype), k2.to(dtype)
    a2, b2 = a.reshape(B * T, HV), b.reshape(B * T, HV)
    g = -torch.exp(A_log.to(dtype)) * softplus(a2.to(dtype) + dt_bias.to(dtype),
                                               softplus_beta, softplus_threshold)
    beta = torch.sigmoid(b2).to(dtype) if ref_rounding else torch.sigmoid(b2.to(dtype))
    vf = v.reshape(B * T, HV, V).to(dtype)
    pool = initial_state.to(dtype).clone()
    out = torch.zeros(B * T, HV, V, dtype=dtype)
    for n in range(cu_seqlens.numel() - 1):
        bos, eos = int(cu_seqlens[n]), int(cu_seqlens[n + 1])
        si = int(state_indices[n])
        h = pool[si].clone() if 0 <= si < pool.shape[0] else torch.zeros(HV, K, V, dtype=dtype)
        for t in range(bos, eos):
            h = h * torch.exp(g[t]).view(HV, 1, 1)
            vc = vf[t] - torch.sum(h * kf[t][:, :, None], dim=1)
            vc = vc * beta[t][:, None]
            h = h + kf[t][:, :, None] * vc[:, None, :]
            out[t] = torch.sum(h * (qf[t] * scale)[:, :, None], dim=1)
        if eos > bos and 0 <= si < pool.shape[0]:
            pool[si] = h
    return out.reshape(B, T, HV, V), pool
