"""Pins for oracle/rope.py (CPU only)."""
import torch
import torch.nn.functional as F

from oracle import rope as orp


def _inputs(T=5, hq=4, hkv=2, hd=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(T, (hq + 2 * hkv) * hd, generator=g, dtype=torch.float64)
    qw = torch.randn(hd, generator=g, dtype=torch.float64) * 0.1 + 1
    kw = torch.randn(hd, generator=g, dtype=torch.float64) * 0.1 + 1
    pos = torch.randint(0, 4096, (T,), generator=g)
    return qkv, qw, kw, pos


def test_rotation_matches_complex_multiplication():
    qkv, qw, kw, pos = _inputs()
    inv = orp.inv_freq_table(64, 1e6)
    cos, sin = orp.neox_cos_sin(pos, inv)
    q, k, _ = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, 256, 128, 64, 1e-6,
                                     dtype=torch.float64)
    qn = F.rms_norm(qkv[:, :256].reshape(5, 4, 64), (64,), qw, eps=1e-6)
    z = torch.complex(qn[..., :32], qn[..., 32:])
    rot = torch.complex(cos[:, None, :32].double(), sin[:, None, :32].double())
    zr = z * rot
    ref = torch.cat([zr.real, zr.imag], -1).reshape(5, 256)
    torch.testing.assert_close(q, ref, rtol=1e-12, atol=1e-12)


def test_pair_norm_preserved_and_v_passthrough():
    qkv, qw, kw, pos = _inputs(seed=1)
    cos, sin = orp.neox_cos_sin(pos, orp.inv_freq_table(64, 1e4))
    q, k, v = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, 256, 128, 64, 1e-6,
                                     dtype=torch.float64)
    kn = F.rms_norm(qkv[:, 256:384].reshape(5, 2, 64), (64,), kw, eps=1e-6)
    kr = k.reshape(5, 2, 64)
    pair = lambda t: t[..., :32] ** 2 + t[..., 32:] ** 2
    # cos/sin are fp32-rounded, so cos^2 + sin^2 = 1 to fp32 precision only
    torch.testing.assert_close(pair(kr), pair(kn), rtol=1e-6, atol=1e-9)
    assert torch.equal(v, qkv[:, 384:])


def test_position_zero_is_plain_rms_norm_with_bias():
    qkv, qw, kw, _ = _inputs(seed=2)
    cos, sin = orp.neox_cos_sin(torch.zeros(5, dtype=torch.long),
                                orp.inv_freq_table(64, 1e6))
    qb = torch.full((64,), 0.25, dtype=torch.float64)
    q, _, _ = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, 256, 128, 64, 1e-6,
                                     q_bias=qb, dtype=torch.float64)
    ref = F.rms_norm(qkv[:, :256].reshape(5, 4, 64), (64,), qw, eps=1e-6) + qb
    torch.testing.assert_close(q, ref.reshape(5, 256))


def test_inv_freq_table_values():
    inv = orp.inv_freq_table(128, 1e6)
    assert inv.shape == (64,)
    assert inv[0] == 1.0
    torch.testing.assert_close(inv[1].double(), torch.tensor(1e6 ** (-2 / 128),
                                                             dtype=torch.float64))
