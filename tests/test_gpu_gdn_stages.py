"""GPU parity of the chunked-GDN stage kernels (a6b-a6g, C-ABI via ops)
against the oracle's stage restatements (oracle/gdn.py, fp32) fed the same
inputs, on varlen tables with empty, one-token and chunk-boundary sequences.

Tolerances: fp32 stage outputs (g_cumsum, A, Ai) rtol 1e-3 / atol 1e-3
(they differ from the oracle by summation order and the ~2^-16 hi/lo-split
products); final states rtol 1e-3 with atol = 1e-3 x RMS(reference); bf16 outputs (w, u, h, v_new, o) rtol 1.6e-2 /
atol 1e-2.  The whole staged pipeline carries the reference's bf16
intermediates (Ai, w, u, h, v_new), so it is compared with the fp32 whole-op
oracle at the reference test's own tolerance, 1e-2 / 1e-2 on o and 2e-2 on
the final state (triton_chunk_gated_delta_rule_test.cpp:46-47).
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as og
from state_tol import assert_state_close

pytestmark = pytest.mark.gpu

F32_TOL = dict(rtol=1e-3, atol=1e-3)
O_TOL = dict(rtol=1.6e-2, atol=1e-2)



def _many(n, seed):
    """cu_seqlens of n sequences of 0..70 tokens (empty, one-token and
    two-chunk ones among them)."""
    lens = torch.randint(0, 71, (n,), generator=torch.Generator().manual_seed(seed))
    return [0] + torch.cumsum(lens, 0).tolist()


# Up to 64 sequences the kernels find their chunks within a wave; past that
# they read the offsets kernel's table (both sides of the switch are here).
CU_CASES = [
    [0, 1, 65, 130, 300],
    [0, 0, 64, 64, 200],
    [0, 4096],
    _many(64, 5),
    _many(80, 6),
]


def _inputs(cu_list, H=2, HV=4, seed=0):
    gen = torch.Generator().manual_seed(seed)
    T = cu_list[-1]
    q = og.l2norm(torch.randn(T, H, 128, generator=gen)).bfloat16()
    k = og.l2norm(torch.randn(T, H, 128, generator=gen)).bfloat16()
    v = torch.randn(T, HV, 128, generator=gen).bfloat16()
    g = F.logsigmoid(torch.randn(T, HV, generator=gen))
    beta = torch.sigmoid(torch.randn(T, HV, generator=gen)).bfloat16()
    h0 = torch.randn(len(cu_list) - 1, HV, 128, 128, generator=gen) * 0.5
    cu = torch.tensor(cu_list, dtype=torch.int32)
    return q, k, v, g, beta, h0, cu


def _b(x, dev):
    return x.unsqueeze(0).to(dev)


@pytest.mark.parametrize("cu_list", CU_CASES)
def test_cumsum(dev, cu_list):
    from torch_npu_ops_amd import ops
    _, _, _, g, _, _, cu = _inputs(cu_list)
    out = ops.npu_chunk_local_cumsum(_b(g, dev), 64, cu.to(dev))[0].cpu()
    ref = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)


def test_cumsum_bf16_batched(dev):
    from torch_npu_ops_amd import ops
    gen = torch.Generator().manual_seed(1)
    g = F.logsigmoid(torch.randn(3, 100, 5, generator=gen)).bfloat16()
    out = ops.npu_chunk_local_cumsum(g.to(dev), 32).cpu()
    ref = torch.cat([og.chunk_local_cumsum(g[b:b + 1].float(), torch.tensor([0, 100]), chunk=32)
                     for b in range(3)])
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("cu_list", CU_CASES)
def test_kkt(dev, cu_list):
    from torch_npu_ops_amd import ops
    _, k, _, g, beta, _, cu = _inputs(cu_list)
    gc = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    A = ops.npu_chunk_scaled_dot_kkt_fwd(_b(k, dev), _b(beta, dev), _b(gc, dev), 64,
                                         cu.to(dev))[0].cpu()
    ref = og.chunk_scaled_dot_kkt(k, beta, gc, cu)
    T = cu_list[-1]
    # rows of tokens inside a sequence only (the reference leaves the rest)
    torch.testing.assert_close(A[:T], ref[:T], **F32_TOL)


@pytest.mark.parametrize("Hg,H", [(4, 4), (1, 4), (3, 6), (2, 10)])
def test_kkt_head_groups(dev, Hg, H):
    """GQA ratios 1, 4 and 2, and head counts that leave a partial group of
    four (the blocks share each qk-head's key tile between its heads)."""
    from torch_npu_ops_amd import ops
    cu_list = [0, 70, 150]
    _, k, _, g, beta, _, cu = _inputs(cu_list, H=Hg, HV=H, seed=4)
    gc = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    A = ops.npu_chunk_scaled_dot_kkt_fwd(_b(k, dev), _b(beta, dev), _b(gc, dev), 64,
                                         cu.to(dev))[0].cpu()
    ref = og.chunk_scaled_dot_kkt(k, beta, gc, cu)
    torch.testing.assert_close(A, ref, **F32_TOL)


@pytest.mark.parametrize("cu_list", CU_CASES)
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_solve_tril(dev, cu_list, out_dtype):
    from torch_npu_ops_amd import ops
    _, k, _, g, beta, _, cu = _inputs(cu_list)
    gc = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    A = og.chunk_scaled_dot_kkt(k, beta, gc, cu)
    Ai = ops.npu_solve_tril(_b(A, dev), 64, cu.to(dev), out_dtype)[0].float().cpu()
    ref = og.solve_tril(A, cu)
    torch.testing.assert_close(Ai, ref, **(F32_TOL if out_dtype == torch.float32 else O_TOL))


@pytest.mark.parametrize("cu_list", CU_CASES)
@pytest.mark.parametrize("ai_dtype", [torch.bfloat16, torch.float32])
def test_recompute_w_u(dev, cu_list, ai_dtype):
    from torch_npu_ops_amd import ops
    _, k, v, g, beta, _, cu = _inputs(cu_list)
    gc = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    Ai = og.solve_tril(og.chunk_scaled_dot_kkt(k, beta, gc, cu), cu).to(ai_dtype)
    w, u = ops.npu_recompute_w_u_fwd(_b(k, dev), _b(v, dev), _b(beta, dev), _b(gc, dev),
                                     _b(Ai, dev), cu.to(dev))
    rw, ru = og.recompute_w_u(k, v, beta, gc, Ai, cu)
    torch.testing.assert_close(w[0].float().cpu(), rw, **O_TOL)
    torch.testing.assert_close(u[0].float().cpu(), ru, **O_TOL)


@pytest.mark.parametrize("cu_list", CU_CASES)
def test_fwd_h(dev, cu_list):
    from torch_npu_ops_amd import ops
    _, k, v, g, beta, h0, cu = _inputs(cu_list)
    gc = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    Ai = og.solve_tril(og.chunk_scaled_dot_kkt(k, beta, gc, cu), cu)
    w, u = og.recompute_w_u(k, v, beta, gc, Ai, cu)
    w, u = w.bfloat16(), u.bfloat16()
    h, vnew, fin = ops.npu_chunk_gated_delta_rule_fwd_h(
        _b(k, dev), _b(w, dev), _b(u, dev), _b(gc, dev), h0.to(dev), True, 64, True, cu.to(dev))
    rh, rv, rf = og.chunk_fwd_h(k, w, u, gc, h0, cu)
    assert h.shape[1] == rh.shape[0]
    torch.testing.assert_close(h[0].float().cpu(), rh, **O_TOL)
    T = cu_list[-1]
    torch.testing.assert_close(vnew[0, :T].float().cpu(), rv[:T], **O_TOL)
    assert_state_close(fin.cpu(), rf)


# V of 32, 64 and 96 (one, two and three 32-column tiles per head).
@pytest.mark.parametrize("V", [32, 64, 96])
def test_fwd_h_v_tiles(dev, V):
    from torch_npu_ops_amd import ops
    cu_list = [0, 1, 65, 130, 300]
    _, k, v, g, beta, h0, cu = _inputs(cu_list)
    v, h0 = v[..., :V].contiguous(), h0[..., :V].contiguous()
    gc = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    Ai = og.solve_tril(og.chunk_scaled_dot_kkt(k, beta, gc, cu), cu)
    w, u = og.recompute_w_u(k, v, beta, gc, Ai, cu)
    w, u = w.bfloat16(), u.bfloat16()
    h, vnew, fin = ops.npu_chunk_gated_delta_rule_fwd_h(
        _b(k, dev), _b(w, dev), _b(u, dev), _b(gc, dev), h0.to(dev), True, 64, True, cu.to(dev))
    rh, rv, rf = og.chunk_fwd_h(k, w, u, gc, h0, cu)
    torch.testing.assert_close(h[0].float().cpu(), rh, **O_TOL)
    torch.testing.assert_close(vnew[0, :300].float().cpu(), rv[:300], **O_TOL)
    assert_state_close(fin.cpu(), rf)


def test_fwd_h_no_decay_no_state(dev):
    from torch_npu_ops_amd import ops
    _, k, v, g, beta, _, cu = _inputs([0, 70, 150])
    gc = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    w, u = og.recompute_w_u(k, v, beta, gc, og.solve_tril(og.chunk_scaled_dot_kkt(k, beta, gc, cu), cu), cu)
    w, u = w.bfloat16(), u.bfloat16()
    h, vnew, fin = ops.npu_chunk_gated_delta_rule_fwd_h(
        _b(k, dev), _b(w, dev), _b(u, dev), None, None, True, 64, False, cu.to(dev))
    assert vnew is None
    rh, _, rf = og.chunk_fwd_h(k, w, u, None, None, cu)
    torch.testing.assert_close(h[0].float().cpu(), rh, **O_TOL)
    assert_state_close(fin.cpu(), rf)


@pytest.mark.parametrize("cu_list", CU_CASES)
def test_fwd_o(dev, cu_list):
    from torch_npu_ops_amd import ops
    q, k, v, g, beta, h0, cu = _inputs(cu_list)
    gc = og.chunk_local_cumsum(g.unsqueeze(0), cu)[0]
    Ai = og.solve_tril(og.chunk_scaled_dot_kkt(k, beta, gc, cu), cu)
    w, u = og.recompute_w_u(k, v, beta, gc, Ai, cu)
    h, vnew, _ = og.chunk_fwd_h(k, w, u, gc, h0, cu)
    h, vnew = h.bfloat16(), vnew.bfloat16()
    o = ops.npu_chunk_fwd_o(_b(q, dev), _b(k, dev), _b(vnew, dev), h.unsqueeze(0).to(dev),
                            _b(gc, dev), 0.0883883, 64, cu.to(dev))
    ro = og.chunk_fwd_o(q, k, vnew, h, gc, 0.0883883, cu)
    T = cu_list[-1]
    torch.testing.assert_close(o[0, :T].float().cpu(), ro[:T], **O_TOL)


@pytest.mark.parametrize("cu_list", [[0, 1, 65, 130, 300], [0, 4096]])
def test_staged_pipeline_matches_whole_op(dev, cu_list):
    """The reference's own composition (npu_triton_chunk_gated_delta_rule.cpp:
    608-642) run stage by stage on the GPU, with its bf16 intermediates."""
    from torch_npu_ops_amd import ops
    q, k, v, g, beta, h0, cu = _inputs(cu_list, seed=3)
    cud = cu.to(dev)
    gc = ops.npu_chunk_local_cumsum(_b(g, dev), 64, cud)
    A = ops.npu_chunk_scaled_dot_kkt_fwd(_b(k, dev), _b(beta, dev), gc, 64, cud)
    Ai = ops.npu_solve_tril(A, 64, cud, torch.bfloat16)
    w, u = ops.npu_recompute_w_u_fwd(_b(k, dev), _b(v, dev), _b(beta, dev), gc, Ai, cud)
    h, vnew, fin = ops.npu_chunk_gated_delta_rule_fwd_h(_b(k, dev), w, u, gc, h0.to(dev), True,
                                                        64, True, cud)
    o = ops.npu_chunk_fwd_o(_b(q, dev), _b(k, dev), vnew, h, gc, 128 ** -0.5, 64, cud)
    ro, rs = og.chunk_gdn(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), g.unsqueeze(0),
                          beta.unsqueeze(0), None, h0, cu)
    torch.testing.assert_close(o.float().cpu(), ro, rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(fin.cpu(), rs, rtol=2e-2, atol=2e-2)
