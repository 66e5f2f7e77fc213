"""Pins for oracle/rope.py (CPU only)."""
import pytest
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


def test_rope_inplace_ref_is_interleaved_complex_rotation():
    # With cos / sin shared by each pair (cos[2i] = cos[2i+1] = cos t_i), the
    # interleaved rotation is (x[2i] + i x[2i+1]) * (cos t_i + i sin t_i).
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(5, 3, 40, generator=gen, dtype=torch.float64)
    t = torch.rand(5, 8, generator=gen, dtype=torch.float64) * 6.0
    cos = torch.cos(t).repeat_interleave(2, -1)
    sin = torch.sin(t).repeat_interleave(2, -1)
    out = orp.rope_inplace_ref(x, sin, cos, 16)
    assert torch.equal(out[..., :24], x[..., :24])
    z = torch.complex(x[..., 24::2], x[..., 25::2]) * torch.polar(
        torch.ones_like(t), t)[:, None, :]
    torch.testing.assert_close(out[..., 24::2].double(), z.real, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(out[..., 25::2].double(), z.imag, rtol=1e-6, atol=1e-6)
    # pair norms are preserved, and cos 1 / sin 0 is the identity
    torch.testing.assert_close(out[..., 24::2] ** 2 + out[..., 25::2] ** 2,
                               x[..., 24::2] ** 2 + x[..., 25::2] ** 2, rtol=1e-6, atol=1e-6)
    ident = orp.rope_inplace_ref(x, torch.zeros(5, 16, dtype=torch.float64),
                                 torch.ones(5, 16, dtype=torch.float64), 16)
    torch.testing.assert_close(ident, x, rtol=1e-7, atol=1e-7)


def test_rope_inplace_ref_uses_each_element_s_own_sin_cos():
    # The reference rotates with per-element sin / cos (not per pair):
    # out[1] = x[1] cos[1] + x[0] sin[1].
    x = torch.tensor([[2.0, 3.0]], dtype=torch.float64)
    out = orp.rope_inplace_ref(x, torch.tensor([[0.5, 0.25]], dtype=torch.float64),
                               torch.tensor([[0.1, 0.2]], dtype=torch.float64), 2)
    # computed in fp32, as the reference does (sin / cos .to(float32))
    assert out[0].tolist() == pytest.approx([2.0 * 0.1 - 3.0 * 0.5, 3.0 * 0.2 + 2.0 * 0.25],
                                            rel=1e-6)
