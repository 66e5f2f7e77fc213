"""CPU restatements of the gated delta rule references (test infrastructure).

recurrent_gdn: torch_recurrent_gated_delta_rule of
  triton_npu/test/triton_recurrent_gated_delta_rule_test.cpp:47-115 (itself a
  port of recurrent_gated_delta_rule_ref, triton_npu/triton_src/
  test_fused_recurrent_gated_delta_rule.py:584-618), run per sequence with
  the GQA expansion and l2norm pre-step of the tests (:697-702; the kernel's
  norm form x/sqrt(sum x^2 + 1e-6), py:131-132), and the slot addressing of
  the kernels (initial state at column accepted-1 with speculative decoding,
  state after token t at column t, py:107-123,155-164,257-307).
chunk_gdn: chunk_gated_delta_rule_full_op_ref of
  triton_npu/test/triton_chunk_gated_delta_rule_test.cpp:190-323 (per
  sequence, per head, per 64-token chunk: WY form with the row-recurrence
  inverse, then the state carry).

Pins (tests/test_oracle_gdn.py): beta = 0 and one-hot-key known answers,
chunked == token-by-token recurrence in float64, the row-recurrence inverse
== torch.linalg.solve_triangular, and per-chunk cumsum == torch.cumsum.
"""
from __future__ import annotations

from typing import Optional

import torch


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x / sqrt(sum(x^2) + eps) over the last dim."""
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def _bounds(cu, N, T):
    if cu is None:
        return [(n * T, (n + 1) * T) for n in range(N)]
    c = [int(v) for v in cu]
    return [(c[i], c[i + 1]) for i in range(len(c) - 1)]


def recurrent_gdn(q, k, v, g, beta, scale: float, state: torch.Tensor,
                  cu_seqlens=None, ssm_state_indices=None,
                  num_accepted_tokens=None, use_qk_l2norm: bool = True,
                  inplace: bool = True, T: Optional[int] = None,
                  dtype=torch.float64):
    """q, k [tokens, H, K]; v [tokens, HV, V]; g, beta [tokens, HV];
    state [slots, HV, K, V] (not modified).  Returns (o [tokens, HV, V],
    new_state) where new_state is the updated pool (inplace) or the dense
    [N, HV, K, V] final states."""
    tokens, H, K = q.shape
    HV, V = v.shape[1], v.shape[2]
    rep = HV // H
    qf, kf = q.to(dtype), k.to(dtype)
    if use_qk_l2norm:
        qf, kf = l2norm(qf), l2norm(kf)
    qf = qf.repeat_interleave(rep, 1) * scale
    kf = kf.repeat_interleave(rep, 1)
    vf, gf = v.to(dtype), g.to(dtype)
    bf = beta.to(dtype) if beta is not None else torch.ones_like(gf)
    N = len(cu_seqlens) - 1 if cu_seqlens is not None else tokens // T
    bounds = _bounds(cu_seqlens, N, T)
    pool = state.to(dtype).clone()
    dense = torch.zeros(N, HV, K, V, dtype=dtype)
    o = torch.zeros(tokens, HV, V, dtype=dtype)
    idx = ssm_state_indices
    per_token = idx is not None and idx.dim() == 2
    for n, (a, b) in enumerate(bounds):
        if b <= a:
            continue
        col0 = int(num_accepted_tokens[n]) - 1 if num_accepted_tokens is not None else 0

        def slot(c):
            if idx is None:
                return n
            return int(idx[n, c]) if idx.dim() == 2 else int(idx[n])
        s0 = slot(col0)
        h = pool[s0].clone() if 0 <= s0 < pool.shape[0] else torch.zeros(HV, K, V, dtype=dtype)
        writes = []
        for i, t in enumerate(range(a, b)):
            h = h * torch.exp(gf[t])[:, None, None]
            vn = bf[t][:, None] * (vf[t] - (h * kf[t][:, :, None]).sum(1))
            h = h + kf[t][:, :, None] * vn[:, None, :]
            o[t] = (h * qf[t][:, :, None]).sum(1)
            if inplace and per_token:
                writes.append((slot(i), h.clone()))
        if inplace:
            if not per_token:
                writes.append((s0, h))
            for sl, hh in writes:
                if 0 <= sl < pool.shape[0]:
                    pool[sl] = hh
        else:
            dense[n] = h
    return o, (pool if inplace else dense)


def chunk_local_cumsum(g: torch.Tensor, cu_seqlens, chunk: int = 64):
    """Per-chunk inclusive cumsum along tokens, restarting each chunk of
    each sequence (BuildChunkLocalCumsum, test.cpp:160-180).  g [1, T, H]."""
    out = torch.zeros_like(g)
    for a, b in _bounds(cu_seqlens, 1, g.shape[1]):
        for s in range(a, b, chunk):
            e = min(s + chunk, b)
            out[:, s:e] = torch.cumsum(g[:, s:e], 1)
    return out


def chunk_gdn(q, k, v, g, beta, scale: Optional[float], initial_state,
              cu_seqlens, chunk: int = 64, use_qk_l2norm: bool = False,
              dtype=torch.float32, heads=None):
    """Chunked gated delta rule of chunk_gated_delta_rule_full_op_ref
    (triton_chunk_gated_delta_rule_test.cpp:190-323).  q, k [1, T, H, K];
    v [1, T, HV, V]; g, beta [1, T, HV]; initial_state [N, HV, K, V] or None.
    Returns (o [1, T, HV, V], final_state [N, HV, K, V]) in `dtype`.
    `heads` restricts the computation to a subset of v-heads (others zero)."""
    _, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    rep = HV // H
    if scale is None:
        scale = K ** -0.5
    qf, kf = q.to(dtype), k.to(dtype)
    if use_qk_l2norm:
        qf, kf = l2norm(qf), l2norm(kf)
    qf = qf.repeat_interleave(rep, 2)[0]
    kf = kf.repeat_interleave(rep, 2)[0]
    vf = v.to(dtype)[0]
    bf = beta.to(dtype)[0]
    gc = chunk_local_cumsum(g.to(dtype), cu_seqlens, chunk)[0]
    bounds = _bounds(cu_seqlens, 1, T)
    o = torch.zeros(T, HV, V, dtype=dtype)
    fin = torch.zeros(len(bounds), HV, K, V, dtype=dtype)
    hs = list(range(HV)) if heads is None else list(heads)
    hi = torch.tensor(hs)
    # The golden loops over heads one at a time; the same per-head algebra
    # is batched over the head dimension here (matmuls per head, the row
    # recurrence stepped for all heads together).
    for n, (a, b) in enumerate(bounds):
        S = (initial_state[n, hi].to(dtype).clone() if initial_state is not None
             else torch.zeros(len(hs), K, V, dtype=dtype))
        for s in range(a, b, chunk):
            e = min(s + chunk, b)
            L = e - s
            qc = qf[s:e, hi].transpose(0, 1) * scale                 # [h, L, K]
            kc = kf[s:e, hi].transpose(0, 1)
            vc = vf[s:e, hi].transpose(0, 1)                         # [h, L, V]
            bc = bf[s:e, hi].transpose(0, 1)                         # [h, L]
            gcc = gc[s:e, hi].transpose(0, 1)
            decay = torch.tril(torch.exp(gcc[:, :, None] - gcc[:, None, :]))
            A = torch.tril(-((kc * bc[..., None]) @ kc.transpose(1, 2)) * decay, -1)
            for r in range(1, L):  # row recurrence, test.cpp:251-257
                A[:, r, :r] = A[:, r, :r] + (A[:, r:r + 1, :r] @ A[:, :r, :r])[:, 0]
            A = A + torch.eye(L, dtype=dtype)
            u = A @ (vc * bc[..., None])
            w = A @ (kc * bc[..., None] * torch.exp(gcc)[..., None])
            attn = torch.tril(qc @ kc.transpose(1, 2) * decay)
            vn = u - w @ S
            o[s:e, hi] = ((qc * torch.exp(gcc)[..., None]) @ S + attn @ vn).transpose(0, 1)
            gl = gcc[:, L - 1]
            S = (S * torch.exp(gl)[:, None, None]
                 + (kc * torch.exp(gl[:, None] - gcc)[..., None]).transpose(1, 2) @ vn)
        fin[n, hi] = S
    return o.unsqueeze(0), fin
