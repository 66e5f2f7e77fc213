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

Stage functions (kkt, solve_tril, recompute_w_u, chunk_fwd_h, chunk_fwd_o)
restate the per-stage kernels of triton_npu/triton_src/chunk_gated_delta_rule
(file:line in each docstring) on the reference's [T, H, ...] layouts.

Pins (tests/test_oracle_gdn.py): beta = 0 and one-hot-key known answers,
chunked == token-by-token recurrence in float64, the row-recurrence inverse
== torch.linalg.solve_triangular, per-chunk cumsum == torch.cumsum, and the
stage functions chained == chunk_gdn in float64 (so a mistake in any stage
changes o or the final state).
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


# ---------------------------------------------------------------------------
# Stage restatements.  Layouts: g, gc, beta [T, H]; q, k [T, Hg, K];
# v, u, v_new, o [T, H, V]; A, Ai [T, H, 64]; w [T, H, K]; h [NT, H, K, V].
# ---------------------------------------------------------------------------
def _safe_exp(x):
    """exp(x) for x <= 0, else 0 (utils.py:82-83)."""
    return torch.where(x <= 0, torch.exp(torch.clamp(x, max=0)), torch.zeros_like(x))


def _seq_chunks(cu, T, chunk=64):
    """(sequence, first token, length) of every chunk, in order."""
    out = []
    for n, (a, b) in enumerate(_bounds(cu, 1, T)):
        for s in range(a, b, chunk):
            out.append((n, s, min(chunk, b - s)))
    return out


def chunk_scaled_dot_kkt(k, beta, gc, cu, dtype=torch.float32):
    """A[t, h, j] = beta_t (k_t . k_{s+j}) exp(gc_t - gc_{s+j}) for j < t - s
    (chunk_scaled_dot_kkt.py:20-86)."""
    T, Hg, K = k.shape
    H = beta.shape[1]
    kf = k.to(dtype).repeat_interleave(H // Hg, 1)
    A = torch.zeros(T, H, 64, dtype=dtype)
    for _, s, L in _seq_chunks(cu, T):
        kc = kf[s:s + L].transpose(0, 1)                      # [H, L, K]
        a = kc @ kc.transpose(1, 2) * beta[s:s + L].to(dtype).t()[:, :, None]
        if gc is not None:
            g = gc[s:s + L].to(dtype).t()
            a = a * _safe_exp(g[:, :, None] - g[:, None, :])
        A[s:s + L, :, :L] = torch.tril(a, -1).transpose(0, 1)
    return A


def solve_tril(A, cu, dtype=torch.float32):
    """Ai = (I + A)^-1 per chunk, by the row recurrence of
    triton_chunk_gated_delta_rule_test.cpp:251-257 applied to -A
    (solve_tril.py computes the same inverse blockwise)."""
    T, H, _ = A.shape
    Ai = torch.zeros(T, H, 64, dtype=dtype)
    for _, s, L in _seq_chunks(cu, T):
        M = -torch.tril(A[s:s + L, :, :L].to(dtype).transpose(0, 1), -1)  # [H, L, L]
        for r in range(1, L):
            M[:, r, :r] = M[:, r, :r] + (M[:, r:r + 1, :r] @ M[:, :r, :r])[:, 0]
        M = M + torch.eye(L, dtype=dtype)
        Ai[s:s + L, :, :L] = M.transpose(0, 1)
    return Ai


def recompute_w_u(k, v, beta, gc, Ai, cu, dtype=torch.float32):
    """u = Ai (v beta), w = Ai (k beta exp(gc)) per chunk (wy_fast.py:21-87)."""
    T, Hg, K = k.shape
    H, V = v.shape[1], v.shape[2]
    kf = k.to(dtype).repeat_interleave(H // Hg, 1)
    w = torch.zeros(T, H, K, dtype=dtype)
    u = torch.zeros(T, H, V, dtype=dtype)
    for _, s, L in _seq_chunks(cu, T):
        a = Ai[s:s + L, :, :L].to(dtype).transpose(0, 1)         # [H, L, L]
        b = beta[s:s + L].to(dtype).t()[:, :, None]
        eg = torch.exp(gc[s:s + L].to(dtype)).t()[:, :, None]
        u[s:s + L] = (a @ (v[s:s + L].to(dtype).transpose(0, 1) * b)).transpose(0, 1)
        w[s:s + L] = (a @ (kf[s:s + L].transpose(0, 1) * b * eg)).transpose(0, 1)
    return w, u


def chunk_fwd_h(k, w, u, gc, h0, cu, dtype=torch.float32):
    """Per sequence and head, per chunk: h[c] = S (entering state),
    v_new = u - w S, S <- exp(gc_last) S + k^T (v_new safe_exp(gc_last - gc))
    (chunk_delta_h.py:22-198).  Returns (h [NT, H, K, V], v_new [T, H, V],
    final [N, H, K, V])."""
    T, Hg, K = k.shape
    H, V = u.shape[1], u.shape[2]
    kf = k.to(dtype).repeat_interleave(H // Hg, 1)
    chunks = _seq_chunks(cu, T)
    bounds = _bounds(cu, 1, T)
    h = torch.zeros(len(chunks), H, K, V, dtype=dtype)
    vnew = torch.zeros(T, H, V, dtype=dtype)
    fin = torch.zeros(len(bounds), H, K, V, dtype=dtype)
    S = {n: (h0[n].to(dtype).clone() if h0 is not None else torch.zeros(H, K, V, dtype=dtype))
         for n in range(len(bounds))}
    for c, (n, s, L) in enumerate(chunks):
        h[c] = S[n]
        vn = u[s:s + L].to(dtype).transpose(0, 1) - w[s:s + L].to(dtype).transpose(0, 1) @ S[n]
        vnew[s:s + L] = vn.transpose(0, 1)
        if gc is not None:
            g = gc[s:s + L].to(dtype).t()                         # [H, L]
            gl = g[:, L - 1]
            vn = vn * _safe_exp(gl[:, None] - g)[:, :, None]
            S[n] = S[n] * torch.exp(gl)[:, None, None]
        S[n] = S[n] + kf[s:s + L].transpose(0, 1).transpose(1, 2) @ vn
    for n in range(len(bounds)):
        fin[n] = S[n]
    return h, vnew, fin


def chunk_fwd_o(q, k, v, h, gc, scale, cu, dtype=torch.float32):
    """o = scale (exp(gc) (q h_c) + tril(q k^T safe_exp(gc_i - gc_j)) v) per
    chunk (chunk_o.py:21-115)."""
    T, Hg, K = q.shape
    H, V = v.shape[1], v.shape[2]
    qf = q.to(dtype).repeat_interleave(H // Hg, 1)
    kf = k.to(dtype).repeat_interleave(H // Hg, 1)
    o = torch.zeros(T, H, V, dtype=dtype)
    for c, (_, s, L) in enumerate(_seq_chunks(cu, T)):
        qc, kc = qf[s:s + L].transpose(0, 1), kf[s:s + L].transpose(0, 1)
        vc = v[s:s + L].to(dtype).transpose(0, 1)
        oc = qc @ h[c].to(dtype)
        a = qc @ kc.transpose(1, 2)
        if gc is not None:
            g = gc[s:s + L].to(dtype).t()
            oc = oc * torch.exp(g)[:, :, None]
            a = a * _safe_exp(g[:, :, None] - g[:, None, :])
        o[s:s + L] = (scale * (oc + torch.tril(a) @ vc)).transpose(0, 1)
    return o
