"""GPU parity of npu_fused_qkvzba_split_reshape_cat (C-ABI via ops, and the
C++ drop-in) against oracle/layout.py on identical seeded inputs.

Cases: every (batch, num_heads_qk, num_heads_v) of
test_fused_qkvzba_split_reshape.py:513-551 (head dims 128, bf16), fp32 / fp16
inputs, odd head dims (scalar path), a row-strided input and the [1, 4]
ratio check of the reference wrapper.  The op is a permutation, so the
outputs must equal the oracle's exactly (the reference test allows 1e-2).
"""
import pytest
import torch

from oracle import layout as ol

pytestmark = pytest.mark.gpu

REF_CASES = [
    (1, 8, 16), (4, 8, 16), (8, 8, 16), (1, 16, 16), (1, 16, 32), (1, 16, 48), (1, 16, 64),
    (4, 16, 32), (8, 16, 32), (64, 16, 16), (64, 8, 8), (64, 4, 4), (64, 2, 2),
    (64, 16, 32), (64, 8, 16), (64, 4, 8), (64, 2, 4), (64, 16, 48), (64, 8, 24),
    (64, 4, 12), (64, 2, 6), (64, 16, 64), (64, 8, 32), (64, 4, 16), (64, 2, 8),
    (4096, 2, 4), (4096, 16, 16), (4096, 4, 8), (4096, 8, 16), (4096, 16, 32),
    (4096, 16, 48), (4096, 16, 64),
]


def _inputs(batch, nqk, nv, hk, hv, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    R = nv // nqk
    qkvz = torch.randn(batch, nqk * (2 * hk + 2 * R * hv), generator=gen).to(dtype)
    ba = torch.randn(batch, nqk * 2 * R, generator=gen).to(dtype)
    return qkvz, ba


def _check(dev, qkvz, ba, nqk, nv, hk, hv, api="ops", qkvz_dev=None):
    if api == "ops":
        from torch_npu_ops_amd import ops as m
    else:
        from torch_npu_ops_amd import _xk_torch as m
    src = qkvz_dev if qkvz_dev is not None else qkvz.to(dev)
    out = m.npu_fused_qkvzba_split_reshape_cat(src, ba.to(dev), nqk, nv, hk, hv)
    torch.cuda.synchronize()
    ref = ol.fused_qkvzba_split_reshape_cat(qkvz, ba, nqk, nv, hk, hv)
    for o, r in zip(out, ref):
        assert o.shape == r.shape and o.dtype == r.dtype
        assert torch.equal(o.cpu(), r)


@pytest.mark.parametrize("batch,nqk,nv", REF_CASES)
def test_reference_cases(dev, batch, nqk, nv):
    _check(dev, *_inputs(batch, nqk, nv, 128, 128, torch.bfloat16, batch + nqk + nv),
           nqk, nv, 128, 128)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_other_dtypes(dev, dtype):
    _check(dev, *_inputs(33, 4, 12, 128, 64, dtype, 1), 4, 12, 128, 64)


def test_odd_head_dims_scalar_path(dev):
    _check(dev, *_inputs(17, 3, 6, 5, 7, torch.bfloat16, 2), 3, 6, 5, 7)


def test_row_strided_input_and_cpp_api(dev):
    qkvz, ba = _inputs(40, 8, 16, 128, 128, torch.bfloat16, 3)
    wide = torch.zeros(40, qkvz.shape[1] + 64, dtype=torch.bfloat16)
    wide[:, 64:] = qkvz
    _check(dev, qkvz, ba, 8, 16, 128, 128, qkvz_dev=wide.to(dev)[:, 64:])
    _check(dev, qkvz, ba, 8, 16, 128, 128, api="cpp")


def test_ratio_above_four_is_refused(dev):
    from torch_npu_ops_amd import _xk_torch as xt
    qkvz, ba = _inputs(2, 2, 10, 8, 8, torch.bfloat16, 4)
    with pytest.raises(RuntimeError, match="v_heads_per_qk in \\[1, 4\\]"):
        xt.npu_fused_qkvzba_split_reshape_cat(qkvz.to(dev), ba.to(dev), 2, 10, 8, 8)
