"""The C++ drop-in API (xllm::kernel::npu / npu_ops over the C-ABI, module
_xk_torch) on the GPU: every entry point gives bit-identical results to the
same kernels driven from Python (ops.py, itself parity-tested against the
oracle), in-place state updates included; the chunked and recurrent GDN ops
are also checked against the oracle directly through this path."""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as og
from state_tol import assert_state_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def xt():
    from torch_npu_ops_amd import _xk_torch
    return _xk_torch


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_layer_norm_paths(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(0)
    x = torch.randn(33, 512, generator=g).bfloat16().to(dev)
    z = torch.randn(33, 512, generator=g).bfloat16().to(dev)
    w = (torch.randn(512, generator=g) * 0.1 + 1).bfloat16().to(dev)
    b = (torch.randn(512, generator=g) * 0.1).bfloat16().to(dev)
    for gs, rms, nbg in ((-1, False, True), (128, True, False), (128, False, True)):
        ref = ops.layer_norm_fwd(x, w, None if rms else b, 1e-5, z, gs, nbg, rms)
        y1 = xt.layer_norm_fwd(x, w, torch.Tensor() if rms else b, 1e-5, z, gs, nbg, rms)
        y2 = xt.npu_ops_layer_norm_fwd(x, w, None if rms else b, 1e-5, z, gs, nbg, rms)
        assert torch.equal(y1, ref) and torch.equal(y2, ref)


def test_gemma_paths(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(1)
    x = torch.randn(2, 17, 1024, generator=g).bfloat16().to(dev)
    gamma = (torch.randn(1024, generator=g) * 0.1).bfloat16().to(dev)
    ry, rr = ops.npu_gemma_rms_norm(x, gamma, 1e-6)
    rstd, y = xt.npu_ops_gemma_rms_norm(x, gamma, 1e-6)
    assert torch.equal(y, ry) and torch.equal(rstd, rr) and rstd.shape == (2, 17, 1)


def test_split_rmsnorm_rope_paths(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(2)
    T, HQ, HKV, D = 19, 8, 2, 128
    qkv = torch.randn(T, (HQ + 2 * HKV) * D, generator=g).to(dev)
    sin, cos = torch.rand(T, D, generator=g).to(dev), torch.rand(T, D, generator=g).to(dev)
    qw, kw = torch.rand(D, generator=g).to(dev), torch.rand(D, generator=g).to(dev)
    ref = ops.npu_split_rmsnorm_rope(qkv, sin, cos, qw, kw, HQ * D, HKV * D, D, 1e-6)
    out = xt.npu_split_rmsnorm_rope(qkv, sin, cos, qw, kw, HQ * D, HKV * D, D, 1e-6)
    for a, b in zip(out, ref):
        assert torch.equal(a, b)


def test_conv_update_paths(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(3)
    x = torch.randn(16, 256, generator=g).bfloat16().to(dev)
    st = torch.randn(20, 256, 3, generator=g).bfloat16().to(dev)
    w = (torch.randn(256, 4, generator=g) * 0.5).bfloat16().to(dev)
    idx = torch.randperm(20, generator=g)[:16].to(torch.int32).to(dev)
    s1, s2 = st.clone(), st.clone()
    ref = ops.npu_causal_conv1d_update(x, s1, w, True, conv_state_indices=idx)
    out = xt.npu_causal_conv1d_update(x, s2, w, True, conv_state_indices=idx)
    assert torch.equal(out, ref) and torch.equal(s1, s2) and not torch.equal(s1, st)


def test_conv_v2_paths(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(4)
    qsl = torch.tensor([0, 5, 70, 71, 200], dtype=torch.int32).to(dev)
    x = torch.randn(200, 384, generator=g).bfloat16().to(dev)
    st = torch.zeros(4, 384, 3, dtype=torch.bfloat16, device=dev)
    w = (torch.randn(384, 4, generator=g) * 0.5).bfloat16().to(dev)
    s1, s2 = st.clone(), st.clone()
    ref = ops.npu_causal_conv1d_update_v2(x, s1, w, True, query_start_loc=qsl)
    out = xt.npu_causal_conv1d_update_v2(x, s2, w, True, query_start_loc=qsl)
    assert torch.equal(out, ref) and torch.equal(s1, s2)


def test_recurrent_paths_and_oracle(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(5)
    B, H, HV, D = 8, 2, 4, 128
    q = torch.randn(1, B, H, D, generator=g).bfloat16()
    k = torch.randn(1, B, H, D, generator=g).bfloat16()
    v = torch.randn(1, B, HV, D, generator=g).bfloat16()
    gate = F.logsigmoid(torch.randn(1, B, HV, generator=g))
    beta = torch.sigmoid(torch.randn(1, B, HV, generator=g)).bfloat16()
    h0 = torch.randn(B, HV, D, D, generator=g) * 0.1
    cu = torch.arange(B + 1, dtype=torch.int32)
    idx = torch.arange(B, dtype=torch.int32)
    d = [t.to(dev) for t in (q, k, v, gate, beta)]
    s1, s2 = h0.to(dev), h0.to(dev)
    o1, f1 = ops.npu_fused_recurrent_gated_delta_rule(*d, 0.1, s1, True, cu.to(dev), idx.to(dev),
                                                      None, True)
    o2, f2 = xt.npu_fused_recurrent_gated_delta_rule(*d, scale=0.1, initial_state=s2,
                                                     cu_seqlens=cu.to(dev),
                                                     ssm_state_indices=idx.to(dev),
                                                     use_qk_l2norm_in_kernel=True)
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    assert f2.data_ptr() == s2.data_ptr()  # in place, the reference's contract
    ro, rs = og.recurrent_gdn(q[0], k[0], v[0], gate[0], beta[0], 0.1, h0, cu, idx)
    torch.testing.assert_close(o2[0].float().cpu(), ro.float(), rtol=1.6e-2, atol=1e-2)
    assert_state_close(s2.cpu(), rs.float())


def test_chunk_paths_and_oracle(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(6)
    cu = torch.tensor([0, 100, 164, 300], dtype=torch.int32)
    T, H, HV = 300, 2, 4
    q = torch.randn(1, T, H, 128, generator=g).bfloat16()
    k = torch.randn(1, T, H, 128, generator=g).bfloat16()
    v = torch.randn(1, T, HV, 128, generator=g).bfloat16()
    gate = F.logsigmoid(torch.randn(1, T, HV, generator=g))
    beta = torch.sigmoid(torch.randn(1, T, HV, generator=g)).bfloat16()
    h0 = torch.randn(3, HV, 128, 128, generator=g)
    d = [t.to(dev) for t in (q, k, v, gate, beta)]
    o1, f1 = ops.npu_chunk_gated_delta_rule(*d, None, h0.to(dev), True, cu.to(dev), False, True)
    o2, f2 = xt.npu_chunk_gated_delta_rule(*d, initial_state=h0.to(dev), output_final_state=True,
                                           cu_seqlens=cu.to(dev), use_qk_l2norm_in_kernel=True)
    assert torch.equal(o1, o2) and torch.equal(f1, f2)
    ro, rs = og.chunk_gdn(q, k, v, gate, beta, None, h0, cu, use_qk_l2norm=True)
    torch.testing.assert_close(o2.float().cpu(), ro, rtol=1.6e-2, atol=1e-2)
    assert_state_close(f2.cpu(), rs)
    # no final state requested: an undefined tensor comes back as None
    _, f3 = xt.npu_chunk_gated_delta_rule(*d, cu_seqlens=cu.to(dev))
    assert f3 is None


def test_chunk_stage_paths(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(7)
    cu = torch.tensor([0, 70, 200], dtype=torch.int32).to(dev)
    T, H, HV = 200, 2, 4
    q = og.l2norm(torch.randn(1, T, H, 128, generator=g)).bfloat16().to(dev)
    k = og.l2norm(torch.randn(1, T, H, 128, generator=g)).bfloat16().to(dev)
    v = torch.randn(1, T, HV, 128, generator=g).bfloat16().to(dev)
    gate = F.logsigmoid(torch.randn(1, T, HV, generator=g)).to(dev)
    beta = torch.sigmoid(torch.randn(1, T, HV, generator=g)).bfloat16().to(dev)
    h0 = torch.randn(2, HV, 128, 128, generator=g).to(dev)
    gc1 = ops.npu_chunk_local_cumsum(gate, 64, cu)
    gc2 = xt.npu_chunk_local_cumsum(gate, 64, cu)
    assert torch.equal(gc1, gc2)
    A1 = ops.npu_chunk_scaled_dot_kkt_fwd(k, beta, gc1, 64, cu)
    A2 = xt.npu_chunk_scaled_dot_kkt_fwd(k, beta, gc1, 64, cu)
    assert torch.equal(A1, A2)
    Ai1 = ops.npu_solve_tril(A1, 64, cu, torch.bfloat16)
    Ai2 = xt.npu_solve_tril(A1, 64, cu, torch.bfloat16)
    assert torch.equal(Ai1, Ai2)
    w1, u1 = ops.npu_recompute_w_u_fwd(k, v, beta, gc1, Ai1, cu)
    w2, u2 = xt.npu_recompute_w_u_fwd(k, v, beta, gc1, Ai1, cu)
    assert torch.equal(w1, w2) and torch.equal(u1, u2)
    h1, vn1, f1 = ops.npu_chunk_gated_delta_rule_fwd_h(k, w1, u1, gc1, h0, True, 64, True, cu)
    h2, vn2, f2 = xt.npu_chunk_gated_delta_rule_fwd_h(k, w1, u1, gc1, h0, True, 64, True, cu)
    assert torch.equal(h1, h2) and torch.equal(vn1, vn2) and torch.equal(f1, f2)
    o1 = ops.npu_chunk_fwd_o(q, k, vn1, h1, gc1, 0.088, 64, cu)
    o2 = xt.npu_chunk_fwd_o(q, k, vn1, h1, gc1, 0.088, 64, cu)
    assert torch.equal(o1, o2)


def test_gdn_conv_decode_paths(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(8)
    B, H, HV, D = 4, 2, 4, 128
    W = 2 * H * D + HV * D
    x = torch.randn(B, W, generator=g).bfloat16().to(dev)
    cs = torch.randn(B, W, 3, generator=g).bfloat16().to(dev)
    cw = (torch.randn(W, 4, generator=g) * 0.5).bfloat16().to(dev)
    gate = (-F.softplus(torch.randn(B, HV, generator=g))).bfloat16().to(dev)
    beta = torch.sigmoid(torch.randn(B, HV, generator=g)).bfloat16().to(dev)
    st = (torch.randn(B, HV, D, D, generator=g) * 0.02).to(dev)
    c1, c2, s1, s2 = cs.clone(), cs.clone(), st.clone(), st.clone()
    o1 = ops.gdn_conv_decode(x, c1, cw, gate, beta, s1, H, HV)
    o2 = xt.npu_gdn_conv_decode(x, c2, cw, gate, beta, s2, H, HV)
    assert torch.equal(o1, o2) and torch.equal(c1, c2) and torch.equal(s1, s2)


def test_recurrent_default_arguments_normalise_like_the_reference(dev, xt):
    # The reference binary always l2-normalises q/k, whatever
    # use_qk_l2norm_in_kernel says (npu_triton_recurrent_gated_delta_rule.cpp:
    # 216-238): a call with default arguments, and one passing False, both
    # match the oracle with the normalisation on.
    g = _g(9)
    B, H, HV, D = 6, 2, 4, 128
    q = torch.randn(1, B, H, D, generator=g).bfloat16()
    k = torch.randn(1, B, H, D, generator=g).bfloat16()
    v = torch.randn(1, B, HV, D, generator=g).bfloat16()
    gate = F.logsigmoid(torch.randn(1, B, HV, generator=g))
    beta = torch.sigmoid(torch.randn(1, B, HV, generator=g)).bfloat16()
    h0 = torch.randn(B, HV, D, D, generator=g) * 0.05
    cu = torch.arange(B + 1, dtype=torch.int32)
    idx = torch.arange(B, dtype=torch.int32)
    ro, rs = og.recurrent_gdn(q[0], k[0], v[0], gate[0], beta[0], D ** -0.5, h0, cu, idx,
                              use_qk_l2norm=True)
    d = [t.to(dev) for t in (q, k, v, gate, beta)]
    for flag in (None, False):
        st = h0.to(dev)
        kw = {} if flag is None else dict(use_qk_l2norm_in_kernel=flag)
        o, _ = xt.npu_fused_recurrent_gated_delta_rule(
            *d, initial_state=st, cu_seqlens=cu.to(dev), ssm_state_indices=idx.to(dev), **kw)
        torch.testing.assert_close(o[0].float().cpu(), ro.float(), rtol=1.6e-2, atol=1e-2)
        assert_state_close(st.cpu(), rs.float())


def test_conv_update_always_applies_silu_like_the_reference(dev, xt):
    # npu_triton_causal_conv1d_update.cpp:38 ignores `activation`: SiLU is
    # built into its kernel.  activation=False still returns the SiLU result.
    from oracle import conv1d as oc
    g = _g(10)
    x = torch.randn(8, 256, generator=g).bfloat16()
    st = torch.randn(8, 256, 3, generator=g).bfloat16()
    w = (torch.randn(256, 4, generator=g) * 0.5).bfloat16()
    idx = torch.arange(8, dtype=torch.int32)
    ry, rst = oc.causal_conv1d_update(x, st, w, None, True, idx)
    for act in (True, False):
        sd = st.to(dev)
        y = xt.npu_causal_conv1d_update(x.to(dev), sd, w.to(dev), act,
                                        conv_state_indices=idx.to(dev))
        torch.testing.assert_close(y.float().cpu(), ry.float(), rtol=1.6e-2, atol=1e-2)
        assert torch.equal(sd.cpu(), rst.to(torch.bfloat16))


def test_sigmoid_gating_update_always_normalises_like_the_reference(dev, xt):
    # The reference wrapper never passes use_qk_l2norm_in_kernel to its
    # kernel, built with the normalisation on: False gives the l2norm result.
    from oracle import gating as ogt
    g = _g(11)
    N, H, HV, D = 4, 2, 4, 128
    q = torch.randn(1, N, H, D, generator=g).bfloat16()
    k = torch.randn(1, N, H, D, generator=g).bfloat16()
    v = torch.randn(1, N, HV, D, generator=g).bfloat16()
    a = torch.randn(1, N, HV, generator=g).bfloat16()
    b = torch.randn(1, N, HV, generator=g).bfloat16()
    A_log = torch.randn(HV, generator=g)
    dt_bias = torch.randn(HV, generator=g)
    h0 = torch.randn(N, HV, D, D, generator=g) * 0.05
    idx = torch.arange(N, dtype=torch.int32)
    cu = torch.arange(N + 1, dtype=torch.int32)
    ro, rs = ogt.sigmoid_gating_delta_rule_update(A_log, a, dt_bias, q, k, v, b, h0, idx, cu,
                                                  D ** -0.5, True)
    st = h0.to(dev)
    o = xt.npu_fused_sigmoid_gating_delta_rule_update(
        A_log.to(dev), a.to(dev), dt_bias.to(dev), q.to(dev), k.to(dev), v.to(dev), b.to(dev),
        st, idx.to(dev), cu.to(dev), use_qk_l2norm_in_kernel=False)
    torch.testing.assert_close(o.float().cpu().reshape(ro.shape), ro.float(), rtol=1.6e-2,
                               atol=1e-2)
    assert_state_close(st.cpu(), rs.float())


def test_gdn_conv_gating_decode_paths(dev, xt):
    from torch_npu_ops_amd import ops
    g = _g(12)
    B, H, HV, D = 4, 2, 4, 128
    W = 2 * H * D + HV * D
    x = torch.randn(B, W, generator=g).bfloat16().to(dev)
    cs = torch.randn(B, W, 3, generator=g).bfloat16().to(dev)
    cw = (torch.randn(W, 4, generator=g) * 0.5).bfloat16().to(dev)
    a = torch.randn(B, HV, generator=g).bfloat16().to(dev)
    b = torch.randn(B, HV, generator=g).bfloat16().to(dev)
    A_log = torch.randn(HV, generator=g).to(dev)
    dt_bias = torch.randn(HV, generator=g).to(dev)
    st = (torch.randn(B, HV, D, D, generator=g) * 0.02).to(dev)
    c1, c2, s1, s2 = cs.clone(), cs.clone(), st.clone(), st.clone()
    o1 = ops.gdn_conv_gating_decode(x, c1, cw, A_log, a, dt_bias, b, s1, H, HV)
    o2 = xt.npu_gdn_conv_sigmoid_gating_decode(x, c2, cw, A_log, a, dt_bias, b, s2, H, HV)
    assert torch.equal(o1, o2) and torch.equal(c1, c2) and torch.equal(s1, s2)
