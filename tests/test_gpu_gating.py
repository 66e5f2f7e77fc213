"""GPU parity of the GDN gating ops (C-ABI via ops, and the C++ drop-in)
against oracle/gating.py on identical seeded inputs.

npu_fused_gdn_gating: the shapes of test_fused_gdn_gating.py:94-107 (tokens
x heads, bf16 a/b, A_log ~N(0,1), dt_bias = 1) and of the gtest
(triton_fused_gdn_gating_test.cpp: 3 tokens, dt_bias ~N(0,1)), plus fp16 /
fp32 inputs and a non-default softplus beta / threshold.  Tolerance: g
within 1e-3 (the reference's), beta_out equal to sigmoid(b) in b's dtype.

npu_fused_sigmoid_gating_delta_rule_update: the (batch, H, HV) list of
test_fused_sigmoid_gating_delta_rule_update.py:225-249 (T = 1, K = V = 128,
l2norm on), varlen multi-token sequences, negative and repeated state
indices and K = V = 64.  Against the kernel-arithmetic oracle (float64):
o (bf16) rtol 1.6e-2 / atol 1e-2, final states (fp32) rtol 1e-3 with atol = 1e-3 x RMS(reference);
against the reference CPU ref's rounding (ref_rounding=True) at that test's
own tolerances (o rtol 5e-3 / atol 1e-2, state rtol 5e-2 / atol 2e-2).
"""
import pytest
import torch

from oracle import gating as og
from state_tol import assert_state_close

pytestmark = pytest.mark.gpu

O_TOL = dict(rtol=1.6e-2, atol=1e-2)

HEADS = (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64)


def _gating_inputs(tokens, heads, dtype, seed, dt_ones=True):
    gen = torch.Generator().manual_seed(seed)
    A_log = torch.randn(heads, generator=gen)
    a = torch.randn(tokens, heads, generator=gen).to(dtype)
    b = torch.randn(tokens, heads, generator=gen).to(dtype)
    dt_bias = torch.ones(heads) if dt_ones else torch.randn(heads, generator=gen)
    return A_log, a, b, dt_bias


def _check_gating(dev, A_log, a, b, dt_bias, beta=1.0, threshold=20.0, api="ops"):
    if api == "ops":
        from torch_npu_ops_amd import ops as api_mod
    else:
        from torch_npu_ops_amd import _xk_torch as api_mod
    g, bo = api_mod.npu_fused_gdn_gating(A_log.to(dev), a.to(dev), b.to(dev), dt_bias.to(dev),
                                         beta, threshold)
    torch.cuda.synchronize()
    rg, rb = og.fused_gdn_gating(A_log, a, b, dt_bias, beta, threshold)
    assert g.shape == rg.shape and g.dtype == torch.float32
    assert bo.shape == rb.shape and bo.dtype == b.dtype
    torch.testing.assert_close(g.cpu(), rg, rtol=1e-3, atol=1e-3)
    torch.testing.assert_close(bo.cpu().float(), rb.float(), rtol=0, atol=1e-3)


@pytest.mark.parametrize("tokens", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("heads", HEADS)
def test_gating_reference_cases(dev, tokens, heads):
    _check_gating(dev, *_gating_inputs(tokens, heads, torch.bfloat16, tokens * 100 + heads))


@pytest.mark.parametrize("heads", HEADS)
def test_gating_gtest_cases(dev, heads):
    _check_gating(dev, *_gating_inputs(3, heads, torch.bfloat16, 42 + heads, dt_ones=False))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_gating_other_dtypes(dev, dtype):
    _check_gating(dev, *_gating_inputs(33, 24, dtype, 5, dt_ones=False))


def test_gating_softplus_beta_and_threshold(dev):
    A_log, a, b, dt_bias = _gating_inputs(64, 32, torch.float32, 6, dt_ones=False)
    a = a * 8  # many values past the threshold branch
    _check_gating(dev, A_log, a, b, dt_bias, beta=2.0, threshold=5.0)


def test_gating_cpp_api(dev):
    _check_gating(dev, *_gating_inputs(16, 32, torch.bfloat16, 7), api="cpp")


def test_gating_large_batch(dev):
    _check_gating(dev, *_gating_inputs(4096, 32, torch.bfloat16, 8, dt_ones=False))


def _every_bf16(lo, hi, heads=32):
    """Every finite bf16 value in [lo, hi], padded with zeros to [rows, heads]."""
    allv = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    f = allv.float()
    vals = allv[torch.isfinite(f) & (f >= lo) & (f <= hi)]
    pad = (-vals.numel()) % heads
    vals = torch.cat([vals, torch.zeros(pad, dtype=torch.bfloat16)])
    return vals.reshape(-1, heads)


def test_gating_softplus_accuracy_every_bf16(dev):
    """g = -softplus(a) (A_log = 0, dt_bias = 0) for every bf16 a in
    [-80, 60]: within 2e-6 relative of the float64 value, a tighter bound
    than the reference's 1e-3; above the threshold g = -a exactly."""
    from torch_npu_ops_amd import ops
    a = _every_bf16(-80.0, 60.0)
    heads = a.shape[1]
    z = torch.zeros(heads)
    g, _ = ops.npu_fused_gdn_gating(z.to(dev), a.to(dev), a.to(dev), z.to(dev), 1.0, 20.0)
    g = g.cpu().double().reshape(a.shape)
    x = a.double()
    ref = -torch.where(x <= 20.0, torch.log1p(torch.exp(x)), x)
    rel = ((g - ref).abs() / ref.abs().clamp_min(1e-300)).max().item()
    assert rel <= 2e-6, rel
    hi = x > 20.0
    assert torch.equal(g[hi], -x[hi])


def test_gating_beta_rounding_every_bf16(dev):
    """beta = sigmoid(b) rounded to bf16 for every bf16 b in [-64, 64]
    (both sides of the kernel's |b| < 32 fast path) equals the correctly
    rounded sigmoid, except where the exact value lies within 4 fp32 ulp of
    a bf16 rounding midpoint (there a 1-ulp fp32 evaluation may round
    either way)."""
    from torch_npu_ops_amd import ops
    b = _every_bf16(-64.0, 64.0)
    heads = b.shape[1]
    z = torch.zeros(heads)
    _, bo = ops.npu_fused_gdn_gating(z.to(dev), b.to(dev), b.to(dev), z.to(dev), 1.0, 20.0)
    bo = bo.cpu().reshape(b.shape)
    s32 = torch.sigmoid(b.double()).float()
    low = s32.view(torch.int32) & 0xFFFF
    near = (low - 0x8000).abs() <= 4
    assert near.float().mean().item() < 1e-3
    ref = s32.bfloat16()
    ok = ~near
    assert torch.equal(bo[ok].view(torch.int16), ref[ok].view(torch.int16))


# ---------------------------------------------------------------------------
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


def _run_update(dev, A_log, a, dt_bias, q, k, v, b, state, idx, cu, scale, l2norm,
                api="ops"):
    if api == "ops":
        from torch_npu_ops_amd import ops as api_mod
    else:
        from torch_npu_ops_amd import _xk_torch as api_mod
    sd = state.to(dev)
    o = api_mod.npu_fused_sigmoid_gating_delta_rule_update(
        A_log.to(dev), a.to(dev), dt_bias.to(dev), q.to(dev), k.to(dev), v.to(dev), b.to(dev),
        sd, idx.to(dev), cu.to(dev), scale, l2norm)
    torch.cuda.synchronize()
    return o.float().cpu(), sd.cpu()


UPDATE_CASES = [(1, 8, 16), (2, 8, 16), (4, 8, 16), (8, 8, 16), (4, 16, 16), (4, 8, 8),
                (4, 4, 4), (4, 2, 2), (4, 16, 32), (4, 4, 8), (4, 2, 4), (4, 16, 48),
                (4, 8, 24), (4, 4, 12), (4, 2, 6), (4, 16, 64), (4, 8, 32), (4, 4, 16),
                (4, 2, 8), (4, 1, 8)]


@pytest.mark.parametrize("batch,H,HV", UPDATE_CASES)
def test_update_reference_cases(dev, batch, H, HV):
    K = V = 128
    q, k, v, a, b, A_log, dt_bias, state = _update_inputs(batch, 1, H, HV, K, V, batch,
                                                          47 + batch + H + HV)
    idx = torch.arange(batch, dtype=torch.int32)
    cu = torch.arange(batch + 1, dtype=torch.int32)
    args = (A_log, a, dt_bias, q, k, v, b, state, idx, cu, K ** -0.5, True)
    o, st = _run_update(dev, *args)
    ro, rs = og.sigmoid_gating_delta_rule_update(*args)
    torch.testing.assert_close(o, ro.float(), **O_TOL)
    assert_state_close(st, rs.float())
    # the reference test's own comparison (its CPU ref rounds beta and q/k)
    fo, fs = og.sigmoid_gating_delta_rule_update(*args, ref_rounding=True)
    torch.testing.assert_close(o, fo.float(), rtol=0.005, atol=0.01)
    torch.testing.assert_close(st, fs.float(), rtol=0.05, atol=0.02)


@pytest.mark.parametrize("l2norm", [True, False])
def test_update_varlen_and_negative_slots(dev, l2norm):
    # One row of 11 tokens: sequences of 3, 0, 1 and 7 tokens; slot 4 is
    # used by none, index -1 starts from zeros and writes nothing.
    K = V = 128
    q, k, v, a, b, A_log, dt_bias, state = _update_inputs(1, 11, 4, 8, K, V, 5, 11)
    q = q * 0.2 if not l2norm else q
    k = k * 0.1 if not l2norm else k
    cu = torch.tensor([0, 3, 3, 4, 11], dtype=torch.int32)
    idx = torch.tensor([2, 0, -1, 3], dtype=torch.int32)
    args = (A_log, a, dt_bias, q, k, v, b, state, idx, cu, 0.3, l2norm)
    o, st = _run_update(dev, *args)
    ro, rs = og.sigmoid_gating_delta_rule_update(*args)
    torch.testing.assert_close(o, ro.float(), **O_TOL)
    assert_state_close(st, rs.float())
    assert torch.equal(st[0], state[0]) and torch.equal(st[1], state[1])
    assert torch.equal(st[4], state[4])


def test_update_head_dim_64_and_cpp_api(dev):
    K = V = 64
    q, k, v, a, b, A_log, dt_bias, state = _update_inputs(6, 1, 2, 4, K, V, 6, 12)
    idx = torch.tensor([5, 4, 3, 2, 1, 0], dtype=torch.int32)
    cu = torch.arange(7, dtype=torch.int32)
    args = (A_log, a, dt_bias, q, k, v, b, state, idx, cu, K ** -0.5, True)
    o, st = _run_update(dev, *args, api="cpp")
    ro, rs = og.sigmoid_gating_delta_rule_update(*args)
    torch.testing.assert_close(o, ro.float(), **O_TOL)
    assert_state_close(st, rs.float())


def test_update_rejects_bad_arguments(dev):
    from torch_npu_ops_amd import ops
    K = V = 128
    q, k, v, a, b, A_log, dt_bias, state = _update_inputs(2, 1, 2, 4, K, V, 2, 13)
    idx = torch.arange(2, dtype=torch.int32)
    cu = torch.arange(3, dtype=torch.int64)  # must be int32
    with pytest.raises(ValueError):
        ops.npu_fused_sigmoid_gating_delta_rule_update(
            A_log.to(dev), a.to(dev), dt_bias.to(dev), q.to(dev), k.to(dev), v.to(dev),
            b.to(dev), state.to(dev), idx.to(dev), cu.to(dev))
