"""Pins for oracle/gdn.py (CPU only): known answers of the recurrence, the
chunked form against the token-by-token recurrence in float64, the
row-recurrence inverse against a triangular solve, and the per-chunk
cumsum against torch.cumsum."""
import torch

from oracle import gdn as og


def _rand(shape, g, scale=1.0):
    return torch.randn(shape, generator=g, dtype=torch.float64) * scale


def test_beta_zero_is_pure_decay():
    g = torch.Generator().manual_seed(0)
    q, k = _rand((1, 2, 16), g), _rand((1, 2, 16), g)
    v = _rand((1, 4, 8), g)
    gate = -torch.rand(1, 4, generator=g, dtype=torch.float64)
    h0 = _rand((1, 4, 16, 8), g)
    o, st = og.recurrent_gdn(q, k, v, gate, torch.zeros(1, 4, dtype=torch.float64),
                             0.5, h0, T=1, ssm_state_indices=torch.tensor([0]))
    hd = h0[0] * torch.exp(gate[0])[:, None, None]
    torch.testing.assert_close(st[0], hd)
    qn = og.l2norm(q[0]).repeat_interleave(2, 0) * 0.5
    torch.testing.assert_close(o[0], torch.einsum("hkv,hk->hv", hd, qn))


def test_one_hot_key_overwrites_row():
    # g = 0, beta = 1, k = e_i (already unit): row i of h becomes v exactly.
    g = torch.Generator().manual_seed(1)
    K, V = 8, 6
    k = torch.zeros(1, 1, K, dtype=torch.float64)
    k[0, 0, 3] = 1
    q = _rand((1, 1, K), g)
    v = _rand((1, 1, V), g)
    h0 = _rand((1, 1, K, V), g)
    _, st = og.recurrent_gdn(q, k, v, torch.zeros(1, 1, dtype=torch.float64),
                             torch.ones(1, 1, dtype=torch.float64), 1.0, h0,
                             T=1, ssm_state_indices=torch.tensor([0]),
                             use_qk_l2norm=False)
    exp = h0[0, 0].clone()
    exp[3] = v[0, 0]
    torch.testing.assert_close(st[0, 0], exp)


def test_chunked_equals_recurrence_float64():
    g = torch.Generator().manual_seed(2)
    T, H, HV, K, V = 150, 2, 4, 16, 8
    q = og.l2norm(_rand((1, T, H, K), g))
    k = og.l2norm(_rand((1, T, H, K), g))
    v = _rand((1, T, HV, V), g)
    gate = -torch.nn.functional.softplus(_rand((1, T, HV), g))
    beta = torch.sigmoid(_rand((1, T, HV), g))
    cu = torch.tensor([0, 70, 71, 150])
    h0 = _rand((3, HV, K, V), g, 0.1)
    oc, fc = og.chunk_gdn(q, k, v, gate, beta, None, h0, cu, chunk=64,
                          dtype=torch.float64)
    orr, fr = og.recurrent_gdn(q[0], k[0], v[0], gate[0], beta[0], K ** -0.5, h0,
                               cu_seqlens=cu, use_qk_l2norm=False, inplace=False)
    torch.testing.assert_close(oc[0], orr, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(fc, fr, rtol=1e-10, atol=1e-10)


def test_row_recurrence_is_the_unit_lower_inverse():
    # The WY inverse of chunk_gated_delta_rule_full_op_ref is (I + A)^-1 for
    # A = tril(beta k k^T decay, -1); compare with a triangular solve.
    g = torch.Generator().manual_seed(3)
    L, K = 64, 32
    kc = og.l2norm(_rand((L, K), g))
    bc = torch.sigmoid(_rand((L,), g))
    gc = torch.cumsum(-torch.rand(L, generator=g, dtype=torch.float64), 0)
    decay = torch.tril(torch.exp(gc[:, None] - gc[None, :]))
    A = torch.tril(-(kc * bc[:, None]) @ kc.t() * decay, -1)
    for r in range(1, L):
        A[r, :r] = A[r, :r] + A[r, :r] @ A[:r, :r]
    A = A + torch.eye(L, dtype=torch.float64)
    M = torch.eye(L, dtype=torch.float64) + torch.tril((kc * bc[:, None]) @ kc.t() * decay, -1)
    ref = torch.linalg.solve_triangular(M, torch.eye(L, dtype=torch.float64), upper=False)
    torch.testing.assert_close(A, ref, rtol=1e-10, atol=1e-12)


def test_chunk_local_cumsum_restarts_per_chunk_and_sequence():
    g = torch.arange(1, 11, dtype=torch.float64).reshape(1, 10, 1)
    out = og.chunk_local_cumsum(g, torch.tensor([0, 3, 10]), chunk=4)
    exp = torch.tensor([1, 3, 6, 4, 9, 15, 22, 8, 17, 27], dtype=torch.float64)
    torch.testing.assert_close(out[0, :, 0], exp)


def test_spec_slots_follow_accepted_tokens():
    g = torch.Generator().manual_seed(4)
    N, T, H, HV, K, V = 2, 3, 1, 2, 8, 4
    q, k = _rand((N * T, H, K), g), _rand((N * T, H, K), g)
    v = _rand((N * T, HV, V), g)
    gate = -torch.rand(N * T, HV, generator=g, dtype=torch.float64)
    beta = torch.sigmoid(_rand((N * T, HV), g))
    pool = _rand((10, HV, K, V), g)
    idx = torch.tensor([[1, 2, 3], [6, 7, 8]])
    acc = torch.tensor([2, 1])
    cu = torch.tensor([0, 3, 6])
    o, st = og.recurrent_gdn(q, k, v, gate, beta, 0.3, pool, cu, idx, acc)
    # sequence 0 starts from slot idx[0, 1] = 2 and writes slots 1, 2, 3
    o0, h0 = og.recurrent_gdn(q[:3], k[:3], v[:3], gate[:3], beta[:3], 0.3,
                              pool[2:3], T=3, ssm_state_indices=torch.tensor([0]))
    torch.testing.assert_close(o[:3], o0)
    torch.testing.assert_close(st[3], h0[0])
    assert torch.equal(st[0], pool[0]) and torch.equal(st[9], pool[9])


def test_stages_chained_equal_whole_op():
    """kkt -> solve_tril -> w/u -> fwd_h -> fwd_o (the reference's stage
    kernels) must reproduce chunk_gdn (pinned against the recurrence above)
    on varlen input with chunk-boundary and one-token sequences."""
    g = torch.Generator().manual_seed(5)
    cu = torch.tensor([0, 1, 65, 130, 200])
    T, H, HV, K, V = 200, 2, 4, 16, 8
    q = og.l2norm(_rand((1, T, H, K), g))
    k = og.l2norm(_rand((1, T, H, K), g))
    v = _rand((1, T, HV, V), g)
    gate = -torch.rand(1, T, HV, generator=g, dtype=torch.float64)
    beta = torch.sigmoid(_rand((1, T, HV), g))
    h0 = _rand((4, HV, K, V), g)
    scale = 0.37
    ref_o, ref_s = og.chunk_gdn(q, k, v, gate, beta, scale, h0, cu, dtype=torch.float64)
    f64 = torch.float64
    gc = og.chunk_local_cumsum(gate, cu)[0]
    A = og.chunk_scaled_dot_kkt(k[0], beta[0], gc, cu, dtype=f64)
    Ai = og.solve_tril(A, cu, dtype=f64)
    w, u = og.recompute_w_u(k[0], v[0], beta[0], gc, Ai, cu, dtype=f64)
    h, vnew, fin = og.chunk_fwd_h(k[0], w, u, gc, h0, cu, dtype=f64)
    o = og.chunk_fwd_o(q[0], k[0], vnew, h, gc, scale, cu, dtype=f64)
    torch.testing.assert_close(o, ref_o[0], rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(fin, ref_s, rtol=1e-10, atol=1e-10)
    # h[c] is the state entering chunk c: the first chunk of each sequence
    # starts from h0, and 4 sequences of lengths 1, 64, 65, 70 give 1+1+2+2.
    assert h.shape[0] == 6
    for c, n in ((0, 0), (1, 1), (2, 2), (4, 3)):
        torch.testing.assert_close(h[c], h0[n])


def test_solve_tril_stage_matches_triangular_solve():
    g = torch.Generator().manual_seed(6)
    T, H = 100, 3
    A = torch.tril(_rand((T, H, 64), g) * 0.3, -1)  # garbage above the diagonal is ignored
    A = A + torch.triu(torch.ones(T, H, 64, dtype=torch.float64), 0) * 7.0
    cu = torch.tensor([0, 40, 100])
    Ai = og.solve_tril(A, cu, dtype=torch.float64)
    for s, L in ((0, 40), (40, 60)):
        for h in range(H):
            m = torch.tril(A[s:s + L, h, :L], -1) + torch.eye(L, dtype=torch.float64)
            ref = torch.linalg.solve_triangular(m, torch.eye(L, dtype=torch.float64), upper=False)
            torch.testing.assert_close(Ai[s:s + L, h, :L], ref, rtol=1e-10, atol=1e-10)
