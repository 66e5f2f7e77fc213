"""Pins of oracle/gating.py (CPU).

softplus / gating are checked against torch.nn.functional.softplus and
values computed with Python's math module; the in-kernel-gating update is
checked against oracle.gdn.recurrent_gdn (pinned by its own known answers in
test_oracle_gdn.py) fed with g and beta from the gating oracle, so a
mistake in the update's loop, its slot handling or its gating plumbing
fails one of them.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gating as og
from oracle import gdn


@pytest.mark.parametrize("beta,threshold", [(1.0, 20.0), (2.0, 20.0), (0.5, 5.0), (1.0, 3.0)])
def test_softplus_matches_torch(beta, threshold):
    x = torch.linspace(-30, 30, 2001, dtype=torch.float64)
    x = torch.cat([x, torch.tensor([threshold / beta, threshold / beta + 1e-9,
                                    threshold / beta - 1e-9], dtype=torch.float64)])
    torch.testing.assert_close(og.softplus(x, beta, threshold),
                               F.softplus(x, beta=beta, threshold=threshold),
                               rtol=1e-12, atol=1e-12)


def test_softplus_known_values():
    x = torch.tensor([0.0, 25.0, 1.5, -40.0], dtype=torch.float64)
    sp = og.softplus(x)
    assert sp[0].item() == pytest.approx(math.log(2.0), rel=1e-15)
    assert sp[1].item() == 25.0  # above the threshold: x itself
    assert sp[2].item() == pytest.approx(math.log1p(math.exp(1.5)), rel=1e-15)
    assert sp[3].item() == pytest.approx(math.exp(-40.0), rel=1e-12)
    # beta scaling: softplus_beta(x) = log(1 + exp(beta x)) / beta
    assert og.softplus(torch.tensor([0.7], dtype=torch.float64), 2.0).item() == pytest.approx(
        math.log1p(math.exp(1.4)) / 2.0, rel=1e-15)


def test_gating_closed_forms():
    a = torch.tensor([[0.0, 0.3, 30.0]], dtype=torch.float64)
    b = torch.tensor([[0.0, 2.0, -2.0]], dtype=torch.float64)
    A_log = torch.tensor([0.0, math.log(3.0), math.log(0.5)], dtype=torch.float64)
    dt_bias = torch.tensor([0.0, 0.2, -1.0], dtype=torch.float64)
    g, s = og.gating(A_log, a, b, dt_bias, dtype=torch.float64)
    assert g[0, 0].item() == pytest.approx(-math.log(2.0), rel=1e-14)
    assert g[0, 1].item() == pytest.approx(-3.0 * math.log1p(math.exp(0.5)), rel=1e-14)
    assert g[0, 2].item() == pytest.approx(-0.5 * 29.0, rel=1e-14)  # threshold branch
    assert s[0, 0].item() == 0.5
    assert s[0, 1].item() + s[0, 2].item() == pytest.approx(1.0, abs=1e-15)
    assert s[0, 1].item() == pytest.approx(1.0 / (1.0 + math.exp(-2.0)), rel=1e-15)


def test_fused_gdn_gating_layout_and_dtypes():
    gen = torch.Generator().manual_seed(0)
    A_log = torch.randn(8, generator=gen)
    dt_bias = torch.ones(8)
    a = torch.randn(3, 8, generator=gen).bfloat16()
    b = torch.randn(3, 8, generator=gen).bfloat16()
    g, beta = og.fused_gdn_gating(A_log, a, b, dt_bias)
    assert g.shape == (1, 3, 8) and g.dtype == torch.float32
    assert beta.shape == (1, 3, 8) and beta.dtype == torch.bfloat16
    # the reference golden evaluates sigmoid in b's dtype
    assert torch.equal(beta[0], b.sigmoid())


def _update_inputs(B, T, H, HV, K, V, slots, seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=gen).bfloat16()
    k = torch.randn(B, T, H, K, generator=gen).bfloat16()
    v = torch.randn(B, T, HV, V, generator=gen).bfloat16()
    a = torch.randn(B, T, HV, generator=gen).bfloat16()
    b = torch.randn(B, T, HV, generator=gen).bfloat16()
    A_log = torch.randn(HV, generator=gen)
    dt_bias = torch.randn(HV, generator=gen)
    state = torch.randn(slots, HV, K, V, generator=gen)
    return q, k, v, a, b, A_log, dt_bias, state


@pytest.mark.parametrize("l2norm", [True, False])
def test_update_equals_recurrent_with_gating(l2norm):
    # One batch row of 7 tokens split into sequences of 2, 0 and 5 tokens;
    # the empty sequence and a negative index must leave their slots alone.
    H, HV, K, V = 2, 4, 8, 6
    q, k, v, a, b, A_log, dt_bias, state = _update_inputs(1, 7, H, HV, K, V, 4, 1)
    cu = torch.tensor([0, 2, 2, 7], dtype=torch.int32)
    idx = torch.tensor([3, 1, -1], dtype=torch.int32)
    o, pool = og.sigmoid_gating_delta_rule_update(A_log, a, dt_bias, q, k, v, b, state, idx,
                                                  cu, 0.37, l2norm)
    g, beta = og.gating(A_log, a[0], b[0], dt_bias, dtype=torch.float64)
    ro, rpool = gdn.recurrent_gdn(q[0], k[0], v[0], g, beta, 0.37, state, cu_seqlens=cu,
                                  ssm_state_indices=idx, use_qk_l2norm=l2norm, inplace=True,
                                  dtype=torch.float64)
    torch.testing.assert_close(o[0], ro, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(pool, rpool, rtol=1e-12, atol=1e-12)
    # slot 3 was updated, 0, 1 and 2 were not (index -1 starts from zeros)
    assert not torch.equal(pool[3], state[3].double())
    for s in (0, 1, 2):
        assert torch.equal(pool[s], state[s].double())


def test_negative_index_starts_from_zero_state():
    H, HV, K, V = 1, 1, 4, 4
    q, k, v, a, b, A_log, dt_bias, state = _update_inputs(1, 1, H, HV, K, V, 2, 2)
    cu = torch.tensor([0, 1], dtype=torch.int32)
    o, _ = og.sigmoid_gating_delta_rule_update(A_log, a, dt_bias, q, k, v, b, state,
                                               torch.tensor([-1], dtype=torch.int32), cu,
                                               1.0, False)
    # From h = 0 one token gives h = beta k v^T and o = h^T q = beta (k.q) v.
    beta = torch.sigmoid(b.double())[0, 0, 0]
    kq = (k.double()[0, 0, 0] * q.double()[0, 0, 0]).sum()
    torch.testing.assert_close(o[0, 0, 0], beta * kq * v.double()[0, 0, 0], rtol=1e-12,
                               atol=1e-12)


def test_ref_rounding_stays_within_the_reference_tolerance():
    H, HV, K, V = 2, 4, 16, 16
    q, k, v, a, b, A_log, dt_bias, state = _update_inputs(2, 1, H, HV, K, V, 2, 3)
    cu = torch.arange(3, dtype=torch.int32)
    idx = torch.arange(2, dtype=torch.int32)
    args = (A_log, a, dt_bias, q, k, v, b, state, idx, cu, K ** -0.5, True)
    o1, s1 = og.sigmoid_gating_delta_rule_update(*args)
    o2, s2 = og.sigmoid_gating_delta_rule_update(*args, ref_rounding=True)
    assert not torch.equal(s1, s2)  # the rounding is really applied
    torch.testing.assert_close(o1, o2, rtol=0.005, atol=0.01)
    torch.testing.assert_close(s1, s2, rtol=0.05, atol=0.02)
