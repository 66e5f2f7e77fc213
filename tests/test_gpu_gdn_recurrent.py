"""GPU parity of the recurrent gated delta rule and the fused conv + GDN
decode step (C-ABI via ops) against oracle/gdn.py (float64) and
oracle/conv1d.py on identical seeded inputs.

Tolerances: outputs (bf16) rtol 1.6e-2 / atol 1e-2; final states (fp32)
rtol 1e-3 with atol = 1e-3 x RMS(reference) (the reference's own
test allows rtol 5e-2 / atol 1e-2, test_fused_recurrent_gated_delta_rule.py:
743-748).  Conv states are copies and must match exactly.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import conv1d as oc
from oracle import gdn as og
from state_tol import assert_state_close

pytestmark = pytest.mark.gpu

O_TOL = dict(rtol=1.6e-2, atol=1e-2)


def _inputs(N, T, H, HV, D, g_norm, seed, gdt=torch.float32):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(N * T, H, D, generator=gen).to(torch.bfloat16)
    k = torch.randn(N * T, H, D, generator=gen).to(torch.bfloat16)
    v = torch.randn(N * T, HV, D, generator=gen).to(torch.bfloat16)
    beta = torch.rand(N * T, HV, generator=gen).to(torch.bfloat16).sigmoid()
    g = (F.logsigmoid(torch.rand(N * T, HV, generator=gen)) / g_norm).to(gdt)
    return q, k, v, g, beta


# (B, T, H, HV, D, scale, gate_logit_normalizer) of
# test_fused_recurrent_gated_delta_rule.py:620-660 (bf16)
REF_CASES = [
    (1, 1, 4, 8, 128, 0.5, 0.1), (2, 1, 4, 8, 128, 0.5, 1), (4, 1, 4, 8, 128, 0.2, 0.1),
    (8, 1, 4, 8, 128, 0.3, 1), (16, 1, 4, 8, 128, 0.2, 1), (32, 1, 4, 8, 128, 0.2, 1),
    (2, 1, 16, 16, 128, 0.2, 1), (2, 1, 8, 8, 128, 0.2, 1), (2, 1, 2, 2, 128, 0.2, 1),
    (2, 1, 16, 32, 128, 0.2, 1), (2, 1, 8, 16, 128, 0.2, 1), (2, 1, 16, 48, 128, 0.2, 1),
    (2, 1, 2, 6, 128, 0.2, 1), (2, 1, 16, 64, 128, 0.2, 1), (2, 1, 2, 8, 128, 0.2, 1),
    (2, 1, 1, 8, 128, 0.2, 1),
]


@pytest.mark.parametrize("B,T,H,HV,D,scale,gn", REF_CASES)
def test_recurrent_reference_cases(dev, B, T, H, HV, D, scale, gn):
    from torch_npu_ops_amd import ops
    q, k, v, g, beta = _inputs(B, T, H, HV, D, gn, 42)
    gen = torch.Generator().manual_seed(7)
    h0 = torch.randn(B, HV, D, D, generator=gen)
    cu = torch.arange(B + 1, dtype=torch.long) * T
    idx = torch.arange(B, dtype=torch.int32)
    ref_o, ref_st = og.recurrent_gdn(q, k, v, g, beta, scale, h0, cu, idx)
    st_d = h0.to(dev)
    o, fin = ops.npu_fused_recurrent_gated_delta_rule(
        q.unsqueeze(0).to(dev), k.unsqueeze(0).to(dev), v.unsqueeze(0).to(dev),
        g.unsqueeze(0).to(dev), beta.unsqueeze(0).to(dev), scale, st_d, True,
        cu.to(dev), idx.to(dev))
    assert fin.data_ptr() == st_d.data_ptr()
    torch.testing.assert_close(o[0].float().cpu(), ref_o.float(), **O_TOL)
    assert_state_close(st_d.cpu(), ref_st.float())


def test_recurrent_config5_unfused(dev):
    # BASELINE config 5 in the unfused a7 form: 256 sequences x 1 token,
    # 16 qk / 32 v heads, bf16 q/k/v/g/beta, state ~N(0, 0.02) in place.
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(0)
    N, H, HV, D = 256, 16, 32, 128
    q = torch.nn.functional.normalize(torch.randn(N, H, D, generator=gen), dim=-1).to(torch.bfloat16)
    k = torch.nn.functional.normalize(torch.randn(N, H, D, generator=gen), dim=-1).to(torch.bfloat16)
    v = torch.randn(N, HV, D, generator=gen).to(torch.bfloat16)
    g = (-F.softplus(torch.randn(N, HV, generator=gen))).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(N, HV, generator=gen)).to(torch.bfloat16)
    h0 = torch.randn(N, HV, D, D, generator=gen) * 0.02
    cu = torch.arange(N + 1, dtype=torch.int32)
    idx = torch.arange(N, dtype=torch.int32)
    ref_o, ref_st = og.recurrent_gdn(q, k, v, g, beta, D ** -0.5, h0, cu, idx)
    st_d = h0.to(dev)
    o, _ = ops.npu_fused_recurrent_gated_delta_rule(
        q.unsqueeze(0).to(dev), k.unsqueeze(0).to(dev), v.unsqueeze(0).to(dev),
        g.unsqueeze(0).to(dev), beta.unsqueeze(0).to(dev), None, st_d, True,
        cu.to(dev), idx.to(dev))
    torch.testing.assert_close(o[0].float().cpu(), ref_o.float(), **O_TOL)
    assert_state_close(st_d.cpu(), ref_st.float())


@pytest.mark.parametrize("case", ["accepted_offsets", "tp4_local"])
def test_recurrent_spec_decoding(dev, case):
    # triton_recurrent_gated_delta_rule_test.cpp:329-567
    from torch_npu_ops_amd import ops
    if case == "accepted_offsets":
        N, T, H, HV, D, scale, pool, seed = 3, 4, 8, 16, 128, 0.5, 32, 44
        idx = torch.tensor([[2, 4, 6, 8], [11, 13, 15, 17], [20, 22, 24, 26]], dtype=torch.int32)
        acc = torch.tensor([1, 2, 3], dtype=torch.int32)
    else:
        N, T, H, HV, D, scale, pool, seed = 8, 2, 1, 8, 128, 0.08838834764831845, 64, 45
        idx = (torch.arange(N * T, dtype=torch.int32).reshape(N, T) + 8)
        acc = torch.tensor([1, 2, 1, 2, 1, 2, 1, 2], dtype=torch.int32)
    q, k, v, g, beta = _inputs(N, T, H, HV, D, 1.0, seed)
    gen = torch.Generator().manual_seed(seed + 1)
    h0 = torch.randn(pool, HV, D, D, generator=gen)
    cu = torch.arange(N + 1, dtype=torch.long) * T
    ref_o, ref_st = og.recurrent_gdn(q, k, v, g, beta, scale, h0, cu, idx, acc)
    st_d = h0.to(dev)
    o, _ = ops.npu_fused_recurrent_gated_delta_rule(
        q.unsqueeze(0).to(dev), k.unsqueeze(0).to(dev), v.unsqueeze(0).to(dev),
        g.unsqueeze(0).to(dev), beta.unsqueeze(0).to(dev), scale, st_d, True,
        cu.to(dev), idx.to(dev), acc.to(dev))
    torch.testing.assert_close(o[0].float().cpu(), ref_o.float(), **O_TOL)
    assert_state_close(st_d.cpu(), ref_st.float())


@pytest.mark.parametrize("K", [64, 128])
def test_recurrent_varlen_not_inplace(dev, K):
    # multi-token sequences (incl. an empty one), int32 cu_seqlens, fp32 g,
    # no beta (= 1), dense final states.
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(3)
    H, HV = 2, 4
    cu = torch.tensor([0, 3, 3, 8, 9], dtype=torch.int32)
    L = 9
    q = torch.randn(1, L, H, K, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, L, H, K, generator=gen).to(torch.bfloat16)
    v = torch.randn(1, L, HV, K, generator=gen).to(torch.bfloat16)
    g = F.logsigmoid(torch.randn(1, L, HV, generator=gen))
    h0 = torch.randn(4, HV, K, K, generator=gen) * 0.1
    ref_o, ref_st = og.recurrent_gdn(q[0], k[0], v[0], g[0], None, 0.3, h0, cu,
                                     None, None, True, inplace=False)
    o, fin = ops.npu_fused_recurrent_gated_delta_rule(
        q.to(dev), k.to(dev), v.to(dev), g.to(dev), None, 0.3, h0.to(dev), False,
        cu.to(dev), None)
    torch.testing.assert_close(o[0].float().cpu(), ref_o.float(), **O_TOL)
    keep = [0, 2, 3]  # sequence 1 is empty: its final state is not written
    assert_state_close(fin.cpu()[keep], ref_st.float()[keep])


def _fused_case(B, H, HV, seed, pad_rows=()):
    gen = torch.Generator().manual_seed(seed)
    D = 2 * H * 128 + HV * 128
    x = torch.randn(B, D, generator=gen).to(torch.bfloat16)
    cs = torch.randn(B, D, 3, generator=gen).to(torch.bfloat16)
    w = (torch.randn(D, 4, generator=gen) * 0.5).to(torch.bfloat16)
    g = (-F.softplus(torch.randn(B, HV, generator=gen))).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, HV, generator=gen)).to(torch.bfloat16)
    st = torch.randn(B, HV, 128, 128, generator=gen) * 0.02
    cidx = torch.arange(B, dtype=torch.int32)
    for r in pad_rows:
        cidx[r] = -1
    return x, cs, w, g, beta, st, cidx


def _fused_ref(x, cs, w, g, beta, st, cidx, H, HV):
    B = x.shape[0]
    y, cs_new = oc.causal_conv1d_update(x, cs, w, None, True, cidx, -1)
    q = y[:, :H * 128].reshape(B, H, 128)
    k = y[:, H * 128:2 * H * 128].reshape(B, H, 128)
    v = y[:, 2 * H * 128:].reshape(B, HV, 128)
    live = [b for b in range(B) if int(cidx[b]) != -1]
    o, st_new = og.recurrent_gdn(q[live], k[live], v[live], g[live], beta[live],
                                 128 ** -0.5, st, T=1,
                                 ssm_state_indices=torch.tensor(live, dtype=torch.int32))
    return live, o, cs_new, st_new


@pytest.mark.parametrize("B,H,HV,pads", [(256, 16, 32, ()), (5, 4, 4, (2,)),
                                          (3, 2, 8, ()), (4, 8, 24, (0, 3))])
def test_fused_conv_decode(dev, B, H, HV, pads):
    # (256, 16, 32) is BASELINE config 5.
    from torch_npu_ops_amd import ops
    x, cs, w, g, beta, st, cidx = _fused_case(B, H, HV, B + H, pads)
    live, ref_o, ref_cs, ref_st = _fused_ref(x, cs, w, g, beta, st, cidx, H, HV)
    cs_d, st_d = cs.to(dev), st.to(dev)
    o = ops.gdn_conv_decode(x.to(dev), cs_d, w.to(dev), g.to(dev), beta.to(dev),
                            st_d, H, HV, conv_state_indices=cidx.to(dev),
                            ssm_state_indices=cidx.clamp(min=0).to(dev))
    torch.testing.assert_close(o[live].float().cpu(), ref_o.float(), **O_TOL)
    assert torch.equal(cs_d.cpu(), ref_cs.to(torch.bfloat16))
    assert_state_close(st_d.cpu(), ref_st.float())


def test_fused_conv_decode_scalar_conv_path(dev):
    # fp32 conv weights and a conv state longer than the window take the
    # per-channel conv path of the fused kernel (not the 8-channel vectors).
    from torch_npu_ops_amd import ops
    B, H, HV = 6, 2, 4
    x, cs, w, g, beta, st, cidx = _fused_case(B, H, HV, 77, (1,))
    live, ref_o, ref_cs, ref_st = _fused_ref(x, cs, w.float(), g, beta, st, cidx, H, HV)
    cs_d, st_d = cs.to(dev), st.to(dev)
    o = ops.gdn_conv_decode(x.to(dev), cs_d, w.float().to(dev), g.to(dev), beta.to(dev),
                            st_d, H, HV, conv_state_indices=cidx.to(dev),
                            ssm_state_indices=cidx.clamp(min=0).to(dev))
    torch.testing.assert_close(o[live].float().cpu(), ref_o.float(), **O_TOL)
    assert torch.equal(cs_d.cpu(), ref_cs.to(torch.bfloat16))
    assert_state_close(st_d.cpu(), ref_st.float())


def _gated_ref(x, cs, w, A_log, a, dt_bias, b, st, cidx, sidx, H, HV):
    """conv1d update + SiLU (oracle/conv1d.py), the [q | k | v] split, then
    the sigmoid-gating recurrent update (oracle/gating.py, kernel arithmetic,
    float64) on the live rows."""
    from oracle import gating as ogt
    B = x.shape[0]
    y, cs_new = oc.causal_conv1d_update(x, cs, w, None, True, cidx, -1)
    live = [r for r in range(B) if int(cidx[r]) != -1]
    q = y[live, :H * 128].reshape(1, len(live), H, 128)
    k = y[live, H * 128:2 * H * 128].reshape(1, len(live), H, 128)
    v = y[live, 2 * H * 128:].reshape(1, len(live), HV, 128)
    o, st_new = ogt.sigmoid_gating_delta_rule_update(
        A_log, a[live][None], dt_bias, q, k, v, b[live][None], st, sidx[live],
        torch.arange(len(live) + 1, dtype=torch.int32), 128 ** -0.5, True)
    return live, o[0], cs_new, st_new


@pytest.mark.parametrize("B,H,HV,pads,neg", [(256, 16, 32, (), ()), (5, 4, 4, (2,), (4,)),
                                              (3, 2, 8, (), (1,)), (4, 8, 24, (0, 3), ())])
def test_fused_conv_gating_decode(dev, B, H, HV, pads, neg):
    # (256, 16, 32) is BASELINE config 5 with the gating in the kernel: the
    # decode step from the projection outputs (mixed_qkv, a, b) in one launch.
    # `neg` rows have a negative state index: zero initial state, no write.
    from torch_npu_ops_amd import ops
    x, cs, w, _, _, st, cidx = _fused_case(B, H, HV, 3 * B + H, pads)
    gen = torch.Generator().manual_seed(B)
    a = torch.randn(B, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(B, HV, generator=gen).to(torch.bfloat16)
    A_log = torch.randn(HV, generator=gen)
    dt_bias = torch.randn(HV, generator=gen)
    sidx = cidx.clamp(min=0)
    for r in neg:
        sidx[r] = -1
    live, ref_o, ref_cs, ref_st = _gated_ref(x, cs, w, A_log, a, dt_bias, b, st, cidx, sidx,
                                             H, HV)
    cs_d, st_d = cs.to(dev), st.to(dev)
    o = ops.gdn_conv_gating_decode(x.to(dev), cs_d, w.to(dev), A_log.to(dev), a.to(dev),
                                   dt_bias.to(dev), b.to(dev), st_d, H, HV,
                                   conv_state_indices=cidx.to(dev),
                                   ssm_state_indices=sidx.to(dev))
    torch.testing.assert_close(o[live].float().cpu(), ref_o.float(), **O_TOL)
    assert torch.equal(cs_d.cpu(), ref_cs.to(torch.bfloat16))
    assert_state_close(st_d.cpu(), ref_st.float())
