"""GPU parity of split_rmsnorm_rope (C-ABI via ops) against oracle/rope.py.

Tolerances: fp32 outputs rtol 1e-5 / atol 1e-5 (same fp32 arithmetic; GPU
sincosf vs CPU sin/cos differ by ~1 ulp); bf16 outputs vs the fp32 oracle
rtol 1.6e-2 / atol 1e-2 (the reference's own pytest
uses atol 5e-2 / rtol 5e-3, test_split_rmsnorm_rope.py:7-8).
"""
import pytest
import torch

from oracle import rope as orp

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-5, atol=1e-5)
BF16_TOL = dict(rtol=1.6e-2, atol=1e-2)


def _case(T, hq, hkv, hd, dtype, seed, theta=1e6, aux=None):
    g = torch.Generator().manual_seed(seed)
    aux = aux or dtype
    qkv = torch.randn(T, (hq + 2 * hkv) * hd, generator=g).to(dtype)
    qw = (torch.randn(hd, generator=g) * 0.1 + 1).to(aux)
    kw = (torch.randn(hd, generator=g) * 0.1 + 1).to(aux)
    pos = torch.randint(0, 4096, (T,), generator=g)
    inv = orp.inv_freq_table(hd, theta)
    cos, sin = orp.neox_cos_sin(pos, inv)
    return qkv, qw, kw, pos, inv, cos.to(aux), sin.to(aux)


def _check(out, ref, dtype):
    tol = F32_TOL if dtype == torch.float32 else BF16_TOL
    for o, r in zip(out, ref):
        torch.testing.assert_close(o.float().cpu(), r, **tol)


def test_config1_tensor_mode(dev):
    # fp32, 256 tokens, 32 q + 8 kv heads, head_dim 128.
    from torch_npu_ops_amd import ops
    qkv, qw, kw, pos, inv, cos, sin = _case(256, 32, 8, 128, torch.float32, 0)
    ref = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, 4096, 1024, 128, 1e-6)
    out = ops.npu_split_rmsnorm_rope(qkv.to(dev), sin.to(dev), cos.to(dev),
                                     qw.to(dev), kw.to(dev), 4096, 1024, 128, 1e-6)
    _check(out, ref, torch.float32)


def test_config1_positions_mode(dev):
    from torch_npu_ops_amd import ops
    qkv, qw, kw, pos, inv, cos, sin = _case(256, 32, 8, 128, torch.float32, 1)
    ref = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, 4096, 1024, 128, 1e-6)
    for pdt in (torch.int64, torch.int32):
        out = ops.npu_split_rmsnorm_rope(qkv.to(dev), None, None, qw.to(dev),
                                         kw.to(dev), 4096, 1024, 128, 1e-6,
                                         positions=pos.to(pdt).to(dev),
                                         inv_freq=inv.to(dev))
        _check(out, ref, torch.float32)


# TP-local head pairs of test_split_rmsnorm_rope.py:10-28 (16/32/64 q heads,
# 8 kv heads over TP 1..16), bf16 as the reference pytest runs them.
@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 4), (4, 2), (2, 1), (1, 1),
                                    (32, 8), (2, 1), (64, 8), (4, 1)])
def test_reference_tp_shapes_bf16(dev, hq, hkv):
    from torch_npu_ops_amd import ops
    qkv, qw, kw, pos, inv, cos, sin = _case(1024, hq, hkv, 128, torch.bfloat16, 0)
    # the reference pytest draws sin/cos ~ N(0,1) (test_split_rmsnorm_rope.py:388-389)
    g = torch.Generator().manual_seed(5)
    sin = torch.randn(1024, 128, generator=g).to(torch.bfloat16)
    cos = torch.randn(1024, 128, generator=g).to(torch.bfloat16)
    ref = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, hq * 128, hkv * 128, 128, 1e-6)
    out = ops.npu_split_rmsnorm_rope(qkv.to(dev), sin.to(dev), cos.to(dev),
                                     qw.to(dev), kw.to(dev), hq * 128, hkv * 128,
                                     128, 1e-6)
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("hd,dtype,aux", [(64, torch.bfloat16, torch.float32),
                                          (256, torch.float16, torch.float16),
                                          (64, torch.float32, torch.float32)])
def test_head_dims_bias_and_aux_dtype(dev, hd, dtype, aux):
    from torch_npu_ops_amd import ops
    qkv, qw, kw, pos, inv, cos, sin = _case(37, 8, 2, hd, dtype, 3, aux=aux)
    g = torch.Generator().manual_seed(9)
    qb = torch.randn(hd, generator=g).to(aux)
    kb = torch.randn(hd, generator=g).to(aux)
    ref = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, 8 * hd, 2 * hd, hd, 1e-6,
                                 q_bias=qb, k_bias=kb)
    out = ops.npu_split_rmsnorm_rope(qkv.to(dev), sin.to(dev), cos.to(dev),
                                     qw.to(dev), kw.to(dev), 8 * hd, 2 * hd, hd,
                                     1e-6, q_bias=qb.to(dev), k_bias=kb.to(dev),
                                     bias=True)
    _check(out, ref, dtype)
    # bias flag off: biases ignored (npu_triton_split_rmsnorm_rope.cpp:109-118)
    ref0 = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, 8 * hd, 2 * hd, hd, 1e-6)
    out0 = ops.npu_split_rmsnorm_rope(qkv.to(dev), sin.to(dev), cos.to(dev),
                                      qw.to(dev), kw.to(dev), 8 * hd, 2 * hd, hd,
                                      1e-6, q_bias=qb.to(dev), k_bias=kb.to(dev),
                                      bias=False)
    _check(out0, ref0, dtype)


# Wave-per-token kernel (from 1024 tokens): 1027 tokens leave a partial last block; 6 q + 3 kv heads give the
# teams of a wave unequal head counts.
@pytest.mark.parametrize("hd,dtype,aux", [(128, torch.bfloat16, torch.bfloat16),
                                          (64, torch.bfloat16, torch.float32),
                                          (256, torch.float16, torch.float16),
                                          (128, torch.float32, torch.float32)])
@pytest.mark.parametrize("mode", ["positions", "table"])
def test_token_kernel(dev, hd, dtype, aux, mode):
    from torch_npu_ops_amd import ops
    T, hq, hkv = 1027, 6, 3
    qkv, qw, kw, pos, inv, cos, sin = _case(T, hq, hkv, hd, dtype, 11, aux=aux)
    g = torch.Generator().manual_seed(12)
    qb = torch.randn(hd, generator=g).to(aux)
    kb = torch.randn(hd, generator=g).to(aux)
    if mode == "positions":
        # the kernel forms cos/sin in fp32, so the oracle gets the fp32 rows
        cos, sin = orp.neox_cos_sin(pos, inv)
    ref = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, hq * hd, hkv * hd, hd, 1e-6,
                                 q_bias=qb, k_bias=kb)
    if mode == "positions":
        out = ops.npu_split_rmsnorm_rope(qkv.to(dev), None, None, qw.to(dev), kw.to(dev),
                                         hq * hd, hkv * hd, hd, 1e-6, q_bias=qb.to(dev),
                                         k_bias=kb.to(dev), bias=True, positions=pos.to(dev),
                                         inv_freq=inv.to(dev))
    else:
        out = ops.npu_split_rmsnorm_rope(qkv.to(dev), sin.to(dev), cos.to(dev), qw.to(dev),
                                         kw.to(dev), hq * hd, hkv * hd, hd, 1e-6,
                                         q_bias=qb.to(dev), k_bias=kb.to(dev), bias=True)
    _check(out, ref, dtype)


# Team kernel (under 1024 tokens): teams of 2 heads when both head counts
# are even, else 1; 301 tokens leave a partial last block.
@pytest.mark.parametrize("hq,hkv", [(32, 8), (12, 4), (6, 2), (10, 2), (5, 1), (3, 3)])
@pytest.mark.parametrize("mode", ["positions", "table"])
def test_team_kernel_head_groups(dev, hq, hkv, mode):
    from torch_npu_ops_amd import ops
    T, hd = 301, 128
    qkv, qw, kw, pos, inv, cos, sin = _case(T, hq, hkv, hd, torch.bfloat16, hq + hkv)
    g = torch.Generator().manual_seed(13)
    qb = torch.randn(hd, generator=g).bfloat16()
    kb = torch.randn(hd, generator=g).bfloat16()
    if mode == "positions":
        cos, sin = orp.neox_cos_sin(pos, inv)
    ref = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, hq * hd, hkv * hd, hd, 1e-6,
                                 q_bias=qb, k_bias=kb)
    kw_ = dict(q_bias=qb.to(dev), k_bias=kb.to(dev), bias=True)
    if mode == "positions":
        out = ops.npu_split_rmsnorm_rope(qkv.to(dev), None, None, qw.to(dev), kw.to(dev),
                                         hq * hd, hkv * hd, hd, 1e-6, positions=pos.to(dev),
                                         inv_freq=inv.to(dev), **kw_)
    else:
        out = ops.npu_split_rmsnorm_rope(qkv.to(dev), sin.to(dev), cos.to(dev), qw.to(dev),
                                         kw.to(dev), hq * hd, hkv * hd, hd, 1e-6, **kw_)
    _check(out, ref, torch.bfloat16)


# Team kernel just under the token-kernel threshold: with fp32 (16-lane
# teams) one CU's share of the 24000 teams exceeds 1024 lanes, so the launch
# uses two blocks per CU; bf16 with head_dim 64 has 4-lane teams.
@pytest.mark.parametrize("dtype,hd", [(torch.float32, 128), (torch.bfloat16, 64)])
def test_team_kernel_many_teams(dev, dtype, hd):
    from torch_npu_ops_amd import ops
    T, hq, hkv = 1000, 32, 8
    qkv, qw, kw, pos, inv, cos, sin = _case(T, hq, hkv, hd, dtype, 21)
    ref = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, hq * hd, hkv * hd, hd, 1e-6)
    out = ops.npu_split_rmsnorm_rope(qkv.to(dev), sin.to(dev), cos.to(dev), qw.to(dev),
                                     kw.to(dev), hq * hd, hkv * hd, hd, 1e-6)
    _check(out, ref, dtype)


def test_single_token_and_empty(dev):
    from torch_npu_ops_amd import ops
    qkv, qw, kw, pos, inv, cos, sin = _case(1, 4, 4, 128, torch.bfloat16, 4)
    ref = orp.split_rmsnorm_rope(qkv, sin, cos, qw, kw, 512, 512, 128, 1e-6)
    out = ops.npu_split_rmsnorm_rope(qkv.to(dev), sin.to(dev), cos.to(dev),
                                     qw.to(dev), kw.to(dev), 512, 512, 128, 1e-6)
    _check(out, ref, torch.bfloat16)
    e = torch.empty(0, 1536, dtype=torch.bfloat16, device=dev)
    es = torch.empty(0, 128, dtype=torch.bfloat16, device=dev)
    q, k, v = ops.npu_split_rmsnorm_rope(e, es, es, qw.to(dev), kw.to(dev), 512,
                                         512, 128, 1e-6)
    assert q.shape == (0, 512) and v.shape == (0, 512)


# rope_inplace: the shapes of test_rope_inplace.py:96-111 (x [batch, head, 512],
# rope_dim 64, bf16 sin / cos [batch, 64]) plus 2-D x, fp32 / fp16, fp32
# sin / cos, odd pair counts (scalar-pair path), strided rows and the C++
# drop-in.  Tolerance: bf16 rtol 1.6e-2 / atol 1e-2 (fp32: 1e-5); the
# untouched prefix must be unchanged bit for bit.
# (37, 12): the wave-per-token kernel's second pass over heads is partial;
# 8 / 16 / 24 / 32 heads take its 1- to 4-pass forms with every row loaded
# first, 40 heads its loop.
@pytest.mark.parametrize("batch,head", [(1, 8), (4, 8), (8, 8), (1, 1), (4, 1), (8, 1),
                                        (4096, 16), (37, 12), (19, 24), (23, 32), (7, 40)])
def test_rope_inplace_reference_cases(dev, batch, head):
    _check_rope_inplace(dev, (batch, head, 512), 64, torch.bfloat16, torch.bfloat16, batch + head)


@pytest.mark.parametrize("shape,rope_dim,dtype,sdtype", [
    ((33, 256), 64, torch.bfloat16, torch.bfloat16),     # 2-D x
    ((7, 4, 128), 128, torch.float32, torch.float32),    # whole row rotated
    ((9, 3, 96), 32, torch.float16, torch.float32),      # fp32 sin / cos
    ((5, 2, 40), 6, torch.bfloat16, torch.bfloat16),     # 3 pairs: pair path
    ((6, 5, 64), 32, torch.float32, torch.float32),      # wave per token, fp32
    ((10, 3, 128), 64, torch.float16, torch.float32),    # wave per token, fp32 sin / cos
])
def test_rope_inplace_shapes(dev, shape, rope_dim, dtype, sdtype):
    _check_rope_inplace(dev, shape, rope_dim, dtype, sdtype, 11)


def test_rope_inplace_cpp_api_and_strided_rows(dev):
    from torch_npu_ops_amd import _xk_torch as xt
    gen = torch.Generator().manual_seed(12)
    base = torch.randn(64, 640, generator=gen).bfloat16()
    sin = torch.randn(64, 64, generator=gen).bfloat16()
    cos = torch.randn(64, 64, generator=gen).bfloat16()
    xd = base.to(dev)
    view = xd[:, 64:576]  # rows of 512 at stride 640
    xt.rope_inplace(view, sin.to(dev), cos.to(dev), 64)
    torch.cuda.synchronize()
    ref = orp.rope_inplace_ref(base[:, 64:576], sin, cos, 64)
    out = xd.cpu()
    assert torch.equal(out[:, :64], base[:, :64]) and torch.equal(out[:, 576:], base[:, 576:])
    torch.testing.assert_close(out[:, 64:576].float(), ref.float(), rtol=1.6e-2, atol=1e-2)


def _check_rope_inplace(dev, shape, rope_dim, dtype, sdtype, seed):
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=gen).to(dtype)
    sin = torch.randn(shape[0], rope_dim, generator=gen).to(sdtype)
    cos = torch.randn(shape[0], rope_dim, generator=gen).to(sdtype)
    xd = x.to(dev)
    ops.rope_inplace(xd, sin.to(dev), cos.to(dev), rope_dim)
    torch.cuda.synchronize()
    ref = orp.rope_inplace_ref(x, sin, cos, rope_dim)
    out = xd.cpu()
    assert torch.equal(out[..., :-rope_dim], x[..., :-rope_dim])
    tol = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=1.6e-2, atol=1e-2)
    torch.testing.assert_close(out.float(), ref.float(), **tol)
