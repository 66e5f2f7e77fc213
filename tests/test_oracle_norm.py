"""Pins for oracle/norm.py against library routines, float64 loops and
invariants (CPU only)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import norm as on


def _np_group_stats(x, G, rms):
    """float64 per-(row, group) loop; returns mean, rstd in group*M+row order."""
    x = x.astype(np.float64)
    M, N = x.shape
    ng = N // G
    mean = np.zeros(ng * M)
    rstd = np.zeros(ng * M)
    for r in range(M):
        for g in range(ng):
            seg = x[r, g * G:(g + 1) * G]
            mu = 0.0 if rms else seg.mean()
            var = ((seg - mu) ** 2).mean()
            mean[g * M + r] = mu
            rstd[g * M + r] = 1.0 / np.sqrt(var + 1e-5)
    return mean, rstd


@pytest.mark.parametrize("rms", [False, True])
def test_layer_norm_matches_torch_routines(rms):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(37, 256, generator=g, dtype=torch.float64)
    w = torch.randn(256, generator=g, dtype=torch.float64)
    b = torch.randn(256, generator=g, dtype=torch.float64)
    y, mean, rstd = on.layer_norm_fwd(x, w, b, 1e-5, is_rms_norm=rms,
                                      dtype=torch.float64)
    if rms:
        ref = F.rms_norm(x, (256,), w, eps=1e-5) + b
        assert mean is None
    else:
        ref = F.layer_norm(x, (256,), w, b, eps=1e-5)
    torch.testing.assert_close(y, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("rms", [False, True])
def test_group_stats_layout_against_float64_loop(rms):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 48, generator=g, dtype=torch.float64) * 3 + 0.5
    w = torch.ones(48, dtype=torch.float64)
    _, mean, rstd = on.layer_norm_fwd(x, w, None, 1e-5, group_size=16,
                                      is_rms_norm=rms, dtype=torch.float64)
    m_ref, r_ref = _np_group_stats(x.numpy(), 16, rms)
    np.testing.assert_allclose(rstd.numpy(), r_ref, rtol=1e-12)
    if not rms:
        np.testing.assert_allclose(mean.numpy(), m_ref, rtol=1e-12, atol=1e-14)


def test_grouped_output_moments():
    # With unit weight and no bias each group of y has mean 0 and biased
    # variance var/(var+eps) -> 1.
    g = torch.Generator().manual_seed(2)
    x = torch.randn(9, 64, generator=g, dtype=torch.float64) * 4 - 1
    y, _, _ = on.layer_norm_fwd(x, torch.ones(64, dtype=torch.float64), None,
                                1e-12, group_size=16, dtype=torch.float64)
    yg = y.reshape(9, 4, 16)
    assert yg.mean(-1).abs().max() < 1e-12
    torch.testing.assert_close(yg.var(-1, unbiased=False),
                               torch.ones(9, 4, dtype=torch.float64),
                               rtol=1e-9, atol=1e-9)


def test_gate_positions():
    # norm_before_gate=True: y = LN(x) * silu(z); False: y = LN(x * silu(z)).
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 32, generator=g, dtype=torch.float64)
    z = torch.randn(4, 32, generator=g, dtype=torch.float64)
    w = torch.randn(32, generator=g, dtype=torch.float64)
    after, _, _ = on.layer_norm_fwd(x, w, None, 1e-6, z=z, norm_before_gate=True,
                                    dtype=torch.float64)
    before, _, _ = on.layer_norm_fwd(x, w, None, 1e-6, z=z,
                                     norm_before_gate=False, dtype=torch.float64)
    torch.testing.assert_close(after, F.layer_norm(x, (32,), w, None, 1e-6) * F.silu(z))
    torch.testing.assert_close(before, F.layer_norm(x * F.silu(z), (32,), w, None, 1e-6))


def test_gemma_reduces_to_rms_norm_with_one_plus_gamma():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, 7, 128, generator=g, dtype=torch.float64)
    gamma = torch.randn(128, generator=g, dtype=torch.float64) * 0.1
    y, rstd = on.gemma_rms_norm(x, gamma, 1e-5, dtype=torch.float64)
    torch.testing.assert_close(y, F.rms_norm(x, (128,), 1 + gamma, eps=1e-5))
    torch.testing.assert_close(
        rstd, torch.rsqrt(x.reshape(-1, 128).pow(2).mean(-1) + 1e-5))


def test_l2norm_unit_norm_and_normalize():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(11, 3, 128, generator=g, dtype=torch.float64)
    y = on.l2norm_last_dim(x, eps=0.0, dtype=torch.float64)
    torch.testing.assert_close(y, F.normalize(x, dim=-1))
    torch.testing.assert_close(y.norm(dim=-1), torch.ones(11, 3, dtype=torch.float64))
