"""GPU parity of the causal conv1d kernels (C-ABI via ops) against
oracle/conv1d.py on identical seeded inputs.

Tolerances: bf16 outputs vs the fp32 oracle rtol 1.6e-2 / atol 1e-2;
fp32 outputs rtol 1e-5 / atol 1e-5.  Conv states are copies of inputs, so
they must match exactly (the reference asserts torch.equal on the state,
test_causal_conv1d_update.py:1254).
"""
import pytest
import torch

from oracle import conv1d as oc

pytestmark = pytest.mark.gpu

BF16_TOL = dict(rtol=1.6e-2, atol=1e-2)
F32_TOL = dict(rtol=1e-5, atol=1e-5)


def _tol(dtype):
    return F32_TOL if dtype == torch.float32 else BF16_TOL


def _rn(shape, g, dtype, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(dtype)


# -- update (decode) ---------------------------------------------------------
@pytest.mark.parametrize("bs", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("dim", [2048, 5120, 2056, 200])
def test_update_reference_cases(dev, bs, dim):
    # test_causal_conv1d_update.py:1213-1255: bf16, width 4, seqlen 1, SiLU,
    # no bias, indices arange.  2056 and 200 channels end in a partial wave
    # (64 lanes x 8 channels), which keeps direct per-lane state accesses.
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(bs * 7 + dim)
    x = _rn((bs, dim, 1), g, torch.bfloat16)
    state = _rn((bs, dim, 3), g, torch.bfloat16)
    w = _rn((dim, 4), g, torch.bfloat16)
    idx = torch.arange(bs, dtype=torch.int32)
    ref, ref_state = oc.causal_conv1d_update(x, state, w, None, True, idx)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update(x.to(dev), st_d, w.to(dev),
                                       conv_state_indices=idx.to(dev))
    torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
    assert torch.equal(st_d.cpu(), ref_state.to(torch.bfloat16))


def test_update_config3_decode(dev):
    # BASELINE config 3b: x [256, 8192], state [256, 8192, 3] ~ N(0,1),
    # w ~ N(0, 0.5), SiLU, indices arange.
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(0)
    x = _rn((256, 8192), g, torch.bfloat16)
    state = _rn((256, 8192, 3), g, torch.bfloat16)
    w = _rn((8192, 4), g, torch.bfloat16, 0.5)
    idx = torch.arange(256, dtype=torch.int32)
    ref, ref_state = oc.causal_conv1d_update(x, state, w, None, True, idx)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update(x.to(dev), st_d, w.to(dev),
                                       conv_state_indices=idx.to(dev))
    torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
    assert torch.equal(st_d.cpu(), ref_state.to(torch.bfloat16))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("W,S,T", [(4, 3, 1), (2, 1, 1), (4, 5, 2), (6, 5, 3),
                                   (3, 4, 1), (1, 2, 2)])
def test_update_generic_shapes(dev, dtype, W, S, T):
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(W * 100 + S * 10 + T)
    B, D, lines = 5, 96, 8
    x = _rn((B, D, T), g, dtype)
    state = _rn((lines, D, S), g, dtype)
    w = _rn((D, W), g, dtype, 0.5)
    b = _rn((D,), g, dtype)
    idx = torch.tensor([6, -1, 2, 0, 7], dtype=torch.int32)  # -1 = pad slot
    ref, ref_state = oc.causal_conv1d_update(x, state, w, b, True, idx, -1)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update(x.to(dev), st_d, w.to(dev), True,
                                       b.to(dev), conv_state_indices=idx.to(dev))
    keep = [0, 2, 3, 4]  # pad rows of the output are not written
    torch.testing.assert_close(out[keep].float().cpu(), ref[keep], **_tol(dtype))
    assert torch.equal(st_d.cpu(), ref_state.to(dtype))


def test_update_fp32_weights_no_activation(dev):
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(11)
    x = _rn((4, 1024), g, torch.bfloat16)
    state = _rn((4, 1024, 3), g, torch.bfloat16)
    w = _rn((1024, 4), g, torch.float32, 0.5)
    ref, ref_state = oc.causal_conv1d_update(x, state, w, None, False)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update(x.to(dev), st_d, w.to(dev), activation=False)
    torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
    assert torch.equal(st_d.cpu(), ref_state.to(torch.bfloat16))


# -- varlen (v2) -------------------------------------------------------------
QWEN_GDN_DIMS = [768, 1024, 1280, 1536, 2048, 2560, 3072, 4096, 5120, 6144,
                 8192, 10240, 12288]  # triton_causal_conv1d_update_v2_test.cpp:340-356


@pytest.mark.parametrize("dim", QWEN_GDN_DIMS)
def test_v2_varlen_apc_decode(dev, dim):
    # triton_causal_conv1d_update_v2_test.cpp:238-315
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(dim)
    B, W = 4, 4
    x = _rn((B, dim), g, torch.bfloat16)
    state = _rn((2 * B, dim, W - 1), g, torch.bfloat16)
    w = _rn((dim, W), g, torch.bfloat16)
    bias = torch.zeros(dim, dtype=torch.bfloat16)
    slots = torch.stack([torch.arange(B), torch.arange(B) + B], 1).int()
    last = torch.ones(B, dtype=torch.int32)
    init = torch.zeros(B, dtype=torch.int32)
    qsl = torch.arange(B + 1, dtype=torch.int32)
    ref, ref_state = oc.causal_conv1d_update_v2(x, state, w, bias, True, slots, qsl,
                                                1, -1, last, init)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update_v2(x.to(dev), st_d, w.to(dev), True,
                                          bias.to(dev), slots.to(dev), qsl.to(dev),
                                          1, -1, last.to(dev), init.to(dev))
    torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
    got = st_d.cpu()
    assert torch.equal(got, ref_state.to(torch.bfloat16))
    assert torch.equal(got[:B], state[:B])          # input slots untouched
    assert not torch.equal(got[B:], state[B:])      # output slots written


def test_v2_dense_no_bias_no_activation(dev):
    # triton_causal_conv1d_update_v2_test.cpp:336-370: batch 2, width 2, seqlen 3
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(5)
    x = _rn((2, 512, 3), g, torch.bfloat16)
    state = _rn((2, 512, 1), g, torch.bfloat16)
    w = _rn((512, 2), g, torch.bfloat16)
    ref, ref_state = oc.causal_conv1d_update_v2(x, state, w, None, False)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update_v2(x.to(dev), st_d, w.to(dev), False)
    torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
    assert torch.equal(st_d.cpu(), ref_state.to(torch.bfloat16))


def test_v2_varlen_pad_width5(dev):
    # triton_causal_conv1d_update_v2_test.cpp:372-446 (pad slot -7, an empty
    # sequence, width 5, max_query_len 3)
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(6)
    dim, W = 1024, 5
    x = _rn((5, dim), g, torch.bfloat16)
    state = _rn((4, dim, W - 1), g, torch.bfloat16)
    w = _rn((dim, W), g, torch.bfloat16)
    bias = torch.zeros(dim, dtype=torch.bfloat16)
    slots = torch.tensor([[0, 1], [-7, -7], [2, 3]], dtype=torch.int32)
    last = torch.tensor([1, 0, 1], dtype=torch.int32)
    init = torch.zeros(3, dtype=torch.int32)
    qsl = torch.tensor([0, 3, 3, 5], dtype=torch.int32)
    ref, ref_state = oc.causal_conv1d_update_v2(x, state, w, bias, True, slots, qsl,
                                                3, -7, last, init)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update_v2(x.to(dev), st_d, w.to(dev), True,
                                          bias.to(dev), slots.to(dev), qsl.to(dev),
                                          3, -7, last.to(dev), init.to(dev))
    torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
    got = st_d.cpu()
    assert torch.equal(got, ref_state.to(torch.bfloat16))
    assert torch.equal(got[0], state[0]) and torch.equal(got[2], state[2])
    assert not torch.equal(got[1], state[1]) and not torch.equal(got[3], state[3])


def _varlen_lengths(n, total, lo, hi, g):
    """8 lengths ~ U{lo..hi} repaired to sum exactly to total."""
    lens = torch.randint(lo, hi + 1, (n,), generator=g)
    diff = total - int(lens.sum())
    i = 0
    while diff != 0:
        j = i % n
        step = max(-(int(lens[j]) - lo), min(hi - int(lens[j]), diff))
        lens[j] += step
        diff -= step
        i += 1
    return lens


@pytest.mark.parametrize("state_rule", [0, 1])
def test_v2_config3_prefill(dev, state_rule):
    # BASELINE config 3a: 8 sequences, 16384 tokens, dim 8192, width 4, SiLU,
    # w ~ N(0, 0.5), zero initial state.
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(0)
    lens = _varlen_lengths(8, 16384, 512, 3584, g)
    qsl = torch.zeros(9, dtype=torch.int32)
    qsl[1:] = torch.cumsum(lens, 0)
    mql = int(lens.max())
    x = _rn((16384, 8192), g, torch.bfloat16)
    w = _rn((8192, 4), g, torch.bfloat16, 0.5)
    state = torch.zeros(8, 8192, 3, dtype=torch.bfloat16)
    ref, ref_state = oc.causal_conv1d_update_v2(x, state, w, None, True, None, qsl,
                                                mql, state_rule=state_rule)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update_v2(x.to(dev), st_d, w.to(dev), True, None,
                                          None, qsl.to(dev), mql,
                                          state_rule=state_rule)
    torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
    assert torch.equal(st_d.cpu(), ref_state.to(torch.bfloat16))


@pytest.mark.parametrize("W", [1, 2, 3, 4, 5, 6])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_v2_varlen_widths_with_history(dev, W, dtype):
    # Sequences shorter and longer than a 32-token tile, tiles that start
    # mid-sequence, empty sequences, an out-of-range slot and nonzero history.
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(W)
    qsl = torch.tensor([0, 1, 40, 40, 75, 140, 141], dtype=torch.int32)
    D = 196  # bf16: not a multiple of 8 -> scalar-channel path; fp32: vectors
    x = _rn((141, D), g, dtype)
    S = max(W - 1, 1) + 1
    state = _rn((7, D, S), g, dtype)
    w = _rn((D, W), g, dtype, 0.5)
    b = _rn((D,), g, dtype)
    slots = torch.tensor([3, 9, 0, 5, 1, 2], dtype=torch.int32)  # 9: out of range
    ref, ref_state = oc.causal_conv1d_update_v2(x, state, w, b, True, slots, qsl, 65)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update_v2(x.to(dev), st_d, w.to(dev), True,
                                          b.to(dev), slots.to(dev), qsl.to(dev), 65)
    torch.testing.assert_close(out.float().cpu(), ref, **_tol(dtype))
    assert torch.equal(st_d.cpu(), ref_state.to(dtype))


def test_v2_spec_decoding(dev):
    # num_accepted_tokens: history at accepted-1, state shift 1
    # (test_causal_conv1d_update_v2.py:94-120, 170-214).
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(9)
    B, T, D, W = 3, 3, 256, 4
    S = W - 1 + T - 1
    x = _rn((B * T, D), g, torch.bfloat16)
    state = _rn((B, D, S), g, torch.bfloat16)
    w = _rn((D, W), g, torch.bfloat16)
    qsl = torch.arange(0, (B + 1) * T, T, dtype=torch.int32)
    acc = torch.tensor([1, 2, 3], dtype=torch.int32)
    idx = torch.arange(B, dtype=torch.int32)
    ref, ref_state = oc.causal_conv1d_update_v2(x, state, w, None, True, idx, qsl, T,
                                                num_accepted_tokens=acc)
    st_d = state.to(dev)
    out = ops.npu_causal_conv1d_update_v2(x.to(dev), st_d, w.to(dev), True, None,
                                          idx.to(dev), qsl.to(dev), T,
                                          num_accepted_tokens=acc.to(dev))
    torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
    assert torch.equal(st_d.cpu(), ref_state.to(torch.bfloat16))


@pytest.mark.parametrize("W", [3, 4, 5, 6])
def test_v2_history_read_next_to_a_tile_edge(dev, W):
    # Sequences starting 1..W-2 tokens before a 16-token tile edge: their
    # first W-1 tokens (whose windows read the conv-state history) straddle
    # the edge.  The final state is written in place into the input slot
    # (in = out), so the history must be read before it is overwritten.
    from torch_npu_ops_amd import ops
    g = torch.Generator().manual_seed(40 + W)
    qsl = torch.tensor([0, 14, 31, 47, 49, 62, 95, 96, 127, 160], dtype=torch.int32)
    D = 256
    B = qsl.numel() - 1
    x = _rn((160, D), g, torch.bfloat16)
    state = _rn((B + 1, D, W - 1), g, torch.bfloat16)
    w = _rn((D, W), g, torch.bfloat16, 0.5)
    slots = torch.randperm(B + 1, generator=g)[:B].to(torch.int32)
    for rule in (0, 1):
        ref, ref_state = oc.causal_conv1d_update_v2(x, state, w, None, True, slots, qsl, 33,
                                                    state_rule=rule)
        st_d = state.to(dev)
        out = ops.npu_causal_conv1d_update_v2(x.to(dev), st_d, w.to(dev), True, None,
                                              slots.to(dev), qsl.to(dev), 33, state_rule=rule)
        torch.testing.assert_close(out.float().cpu(), ref, **BF16_TOL)
        assert torch.equal(st_d.cpu(), ref_state.to(torch.bfloat16))
