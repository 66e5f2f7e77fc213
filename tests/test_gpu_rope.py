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
