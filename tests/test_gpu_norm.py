"""GPU parity of the normalisation kernels (C-ABI via torch_npu_ops_amd.ops)
against oracle/norm.py on identical seeded inputs.

Tolerances: bf16/f16 outputs vs the fp32 oracle rtol 1.6e-2 / atol 1e-2;
fp32 outputs max-abs 1e-3 (triton_layernorm_fwd_test.cpp:34); fp32 stats
rtol 1e-4 / atol 1e-5 (same fp32 arithmetic, different summation order).
"""
import pytest
import torch

from oracle import norm as on

pytestmark = pytest.mark.gpu

BF16_TOL = dict(rtol=1.6e-2, atol=1e-2)
F32_TOL = dict(rtol=0.0, atol=1e-3)
STAT_TOL = dict(rtol=1e-4, atol=1e-5)


def _tol(dtype):
    return F32_TOL if dtype == torch.float32 else BF16_TOL


def _rand(shape, gen, dtype, scale=1.0, shift=0.0):
    return (torch.randn(shape, generator=gen) * scale + shift).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("has_bias,has_z,gate,rms", [
    (True, False, True, False), (False, False, True, True),
    (True, False, True, True), (True, True, True, False),
    (False, True, True, True), (True, True, False, False),
    (False, True, False, True),
])
def test_layer_norm_reference_cases(dev, dtype, has_bias, has_z, gate, rms):
    # Shapes of test_layernorm_fwd.py:1568-1584 (batch*seq rows, feat 128).
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(42)
    x = _rand((2, 8, 128), gen, dtype)
    w = _rand((128,), gen, dtype)
    b = _rand((128,), gen, dtype) if has_bias else None
    z = _rand((2, 8, 128), gen, dtype) if has_z else None
    ref, rmean, rrstd = on.layer_norm_fwd(x, w, b, 1e-6, z=z, norm_before_gate=gate,
                                          is_rms_norm=rms)
    y, mean, rstd = ops.layer_norm_fwd(
        x.to(dev), w.to(dev), b.to(dev) if b is not None else None, 1e-6,
        z=z.to(dev) if z is not None else None, group_size=128,
        norm_before_gate=gate, is_rms_norm=rms, return_stats=True)
    torch.testing.assert_close(y.float().cpu(), ref, **_tol(dtype))
    torch.testing.assert_close(rstd.cpu(), rrstd, **STAT_TOL)
    if not rms:
        torch.testing.assert_close(mean.cpu(), rmean, **STAT_TOL)


@pytest.mark.parametrize("M,N,G,dtype", [
    (32768, 128, 128, torch.float32),    # test_layernorm_fwd.py:1570
    (1024, 128, 128, torch.bfloat16),    # nomask AOT case, :1614
    (112, 1024, 128, torch.float32),     # ngroups = 8
    (7, 4096, 1024, torch.bfloat16),     # ngroups = 4, TPG 64
    (5, 100, 50, torch.bfloat16),        # unaligned: scalar path
    (3, 65536, 65536, torch.bfloat16),   # group beyond one register tile
    (2, 24576, 8192, torch.float32),     # stream path for fp32
])
def test_layer_norm_shapes(dev, M, N, G, dtype):
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(7)
    x = _rand((M, N), gen, dtype, 2.0, 0.3)
    z = _rand((M, N), gen, dtype)
    w = _rand((N,), gen, dtype, 0.1, 1.0)
    b = _rand((N,), gen, dtype, 0.1)
    for rms in (False, True):
        ref, rmean, rrstd = on.layer_norm_fwd(x, w, b, 1e-5, z=z, group_size=G,
                                              is_rms_norm=rms)
        y, mean, rstd = ops.layer_norm_fwd(x.to(dev), w.to(dev), b.to(dev), 1e-5,
                                           z=z.to(dev), group_size=G,
                                           is_rms_norm=rms, return_stats=True)
        torch.testing.assert_close(y.float().cpu(), ref, **_tol(dtype))
        torch.testing.assert_close(rstd.cpu(), rrstd, **STAT_TOL)
        if not rms:
            torch.testing.assert_close(mean.cpu(), rmean, **STAT_TOL)


@pytest.mark.parametrize("G,dtype", [
    (16, torch.bfloat16), (40, torch.bfloat16), (64, torch.bfloat16), (96, torch.bfloat16),
    (128, torch.bfloat16), (256, torch.bfloat16), (512, torch.bfloat16),
    (16, torch.float32), (64, torch.float32), (128, torch.float32), (256, torch.float32),
])
def test_layer_norm_narrow_groups(dev, G, dtype):
    # Every narrow-group team shape (4 / 8 / 16 / 32 lanes x 2 vectors),
    # full and masked, with and without the gate on either side of the norm.
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(G)
    M, N = 300, 3 * G
    x = _rand((M, N), gen, dtype, 2.0, 0.3)
    z = _rand((M, N), gen, dtype)
    w = _rand((N,), gen, dtype, 0.1, 1.0)
    for rms, gate, zz in ((False, True, None), (True, True, z), (True, False, z)):
        ref, rmean, rrstd = on.layer_norm_fwd(x, w, None, 1e-6, z=zz, group_size=G,
                                              norm_before_gate=gate, is_rms_norm=rms)
        y, mean, rstd = ops.layer_norm_fwd(x.to(dev), w.to(dev), None, 1e-6,
                                           z=zz.to(dev) if zz is not None else None,
                                           group_size=G, norm_before_gate=gate,
                                           is_rms_norm=rms, return_stats=True)
        torch.testing.assert_close(y.float().cpu(), ref, **_tol(dtype))
        torch.testing.assert_close(rstd.cpu(), rrstd, **STAT_TOL)
        if not rms:
            torch.testing.assert_close(mean.cpu(), rmean, **STAT_TOL)


def test_gated_rms_norm_epilogue(dev):
    # The GDN output norm (the reference's nomask kernel shape,
    # test_layernorm_fwd.py:1614-1638, scaled up): rows of one 128-wide
    # head, RMS, gate applied after the norm, no bias, bf16.
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(9)
    M = 131072
    x = _rand((M, 128), gen, torch.bfloat16, 0.5)
    z = _rand((M, 128), gen, torch.bfloat16, 0.5)
    w = _rand((128,), gen, torch.bfloat16, 0.5)
    ref, _, rrstd = on.layer_norm_fwd(x, w, None, 1e-6, z=z, group_size=128,
                                      norm_before_gate=True, is_rms_norm=True)
    y, _, rstd = ops.layer_norm_fwd(x.to(dev), w.to(dev), None, 1e-6, z=z.to(dev),
                                    group_size=128, norm_before_gate=True, is_rms_norm=True,
                                    return_stats=True)
    torch.testing.assert_close(y.float().cpu(), ref, **BF16_TOL)
    torch.testing.assert_close(rstd.cpu(), rrstd, **STAT_TOL)


def test_layer_norm_strided_rows(dev):
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(8)
    base = _rand((64, 384), gen, torch.bfloat16)
    x = base[:, 64:320]  # row stride 384, 16-byte aligned
    w = _rand((256,), gen, torch.bfloat16, 0.1, 1.0)
    ref, _, _ = on.layer_norm_fwd(x, w, None, 1e-5)
    y = ops.layer_norm_fwd(base.to(dev)[:, 64:320], w.to(dev), None, 1e-5)
    torch.testing.assert_close(y.float().cpu(), ref, **BF16_TOL)


def test_layer_norm_config2_full_size(dev):
    # BASELINE config 2a: bf16 16384 x 4096, w ~ N(1, 0.1), b ~ N(0, 0.1).
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(0)
    x = _rand((16384, 4096), gen, torch.bfloat16)
    w = _rand((4096,), gen, torch.bfloat16, 0.1, 1.0)
    b = _rand((4096,), gen, torch.bfloat16, 0.1)
    ref, rmean, rrstd = on.layer_norm_fwd(x, w, b, 1e-5)
    y, mean, rstd = ops.layer_norm_fwd(x.to(dev), w.to(dev), b.to(dev), 1e-5,
                                       return_stats=True)
    torch.testing.assert_close(y.float().cpu(), ref, **BF16_TOL)
    torch.testing.assert_close(mean.cpu(), rmean, **STAT_TOL)
    torch.testing.assert_close(rstd.cpu(), rrstd, **STAT_TOL)


@pytest.mark.parametrize("shape,dtype", [
    ((16384, 4096), torch.bfloat16),   # BASELINE config 2b
    ((3, 5, 128), torch.float32),
    ((9, 1000), torch.bfloat16),
])
def test_gemma_rms_norm(dev, shape, dtype):
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(1)
    x = _rand(shape, gen, dtype)
    gamma = _rand((shape[-1],), gen, dtype, 0.1, 1.0)
    ref, rrstd = on.gemma_rms_norm(x, gamma, 1e-5)
    y, rstd = ops.npu_gemma_rms_norm(x.to(dev), gamma.to(dev), 1e-5)
    torch.testing.assert_close(y.float().cpu(), ref, **_tol(dtype))
    assert rstd.shape == tuple(shape[:-1]) + (1,)
    torch.testing.assert_close(rstd.reshape(-1).cpu(), rrstd, **STAT_TOL)


@pytest.mark.parametrize("shape", [(1, 31, 4, 64), (1, 31, 4, 128),
                                   (2, 17, 3, 192), (2, 64, 8, 256)])
def test_l2norm_reference_shapes(dev, shape):
    # Shapes of test_l2norm.py:97-99.
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(2)
    x = _rand(shape, gen, torch.bfloat16)
    ref = on.l2norm_last_dim(x)
    y = ops.npu_l2norm_last_dim(x.to(dev))
    assert y.dtype == torch.bfloat16
    torch.testing.assert_close(y.float().cpu(), ref, **BF16_TOL)
    y32 = ops.npu_l2norm_last_dim(x.to(dev), output_dtype=torch.float32)
    torch.testing.assert_close(y32.cpu(), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("cols,dtype", [(8, torch.bfloat16), (128, torch.bfloat16),
                                        (136, torch.bfloat16), (2048, torch.bfloat16),
                                        (4096, torch.bfloat16), (100, torch.bfloat16),
                                        (128, torch.float32), (1000, torch.float32),
                                        (64, torch.float16)])
def test_l2norm_row_widths(dev, cols, dtype):
    # Every team width of the vector path (8 .. 2048 elements per 16-bit row,
    # 128 and 1000 per fp32 row; 136 and 1000 leave lanes masked), and the
    # per-row fallback for rows wider than 256 vectors (4096) or not a whole
    # number of 16-byte vectors (100).
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(3)
    x = _rand((301, cols), gen, dtype)
    ref = on.l2norm_last_dim(x)
    y = ops.npu_l2norm_last_dim(x.to(dev), output_dtype=torch.float32)
    torch.testing.assert_close(y.cpu(), ref, rtol=1e-5, atol=1e-6)
    yb = ops.npu_l2norm_last_dim(x.to(dev))
    assert yb.dtype == dtype
    torch.testing.assert_close(yb.float().cpu(), ref, **BF16_TOL)
