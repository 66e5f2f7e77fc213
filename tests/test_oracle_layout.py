"""Pins of oracle/layout.py (CPU): the split is a permutation, checked with
index-valued inputs against hand-worked positions, a bijection check and the
element-by-element restatement of the group layout."""
import pytest
import torch

from oracle import layout as ol


def _index_inputs(rows, nqk, nv, hk, hv):
    R = nv // nqk
    w = nqk * (2 * hk + 2 * R * hv)
    qkvz = torch.arange(rows * w, dtype=torch.float64).reshape(rows, w)
    ba = torch.arange(rows * 2 * nv, dtype=torch.float64).reshape(rows, 2 * nv)
    return qkvz, ba, w


def test_hand_worked_positions():
    # 2 qk heads, 4 v heads (R = 2), head_qk 3, head_v 2: group width
    # 3 + 3 + 4 + 4 = 14, row = [g0: q0 q1 q2 k0 k1 k2 v00 v01 v10 v11 z.. | g1: ...]
    qkvz, ba, w = _index_inputs(1, 2, 4, 3, 2)
    qkv, z, b, a = ol.fused_qkvzba_split_reshape_cat(qkvz, ba, 2, 4, 3, 2)
    assert qkv[0].tolist() == [0, 1, 2, 14, 15, 16,        # q of groups 0, 1
                               3, 4, 5, 17, 18, 19,        # k of groups 0, 1
                               6, 7, 8, 9, 20, 21, 22, 23]  # v heads 0..3
    assert z[0].tolist() == [[10, 11], [12, 13], [24, 25], [26, 27]]
    assert b[0].tolist() == [0, 1, 4, 5] and a[0].tolist() == [2, 3, 6, 7]


@pytest.mark.parametrize("nqk,nv,hk,hv", [(2, 2, 4, 4), (2, 4, 8, 4), (1, 3, 5, 6),
                                          (4, 16, 8, 8), (16, 64, 128, 128)])
def test_bijection_and_elementwise_restatement(nqk, nv, hk, hv):
    rows = 3
    qkvz, ba, w = _index_inputs(rows, nqk, nv, hk, hv)
    qkv, z, b, a = ol.fused_qkvzba_split_reshape_cat(qkvz, ba, nqk, nv, hk, hv)
    sq, sz, sb, sa = ol.source_of(nqk, nv, hk, hv)
    base = torch.arange(rows, dtype=torch.float64)[:, None]
    assert torch.equal(qkv, base * w + torch.tensor(sq, dtype=torch.float64))
    assert torch.equal(z.reshape(rows, -1), base * w + torch.tensor(sz, dtype=torch.float64))
    assert torch.equal(b, base * 2 * nv + torch.tensor(sb, dtype=torch.float64))
    assert torch.equal(a, base * 2 * nv + torch.tensor(sa, dtype=torch.float64))
    # every source element appears exactly once
    got = torch.cat([qkv.reshape(-1), z.reshape(-1)]).sort().values
    assert torch.equal(got, qkvz.reshape(-1))
    assert torch.equal(torch.cat([b.reshape(-1), a.reshape(-1)]).sort().values, ba.reshape(-1))


def test_dtypes_are_kept():
    qkvz = torch.randn(2, 2 * (8 + 8)).bfloat16()  # 2 groups x (q 4 + k 4 + v 4 + z 4)
    ba = torch.randn(2, 8).half()
    qkv, z, b, a = ol.fused_qkvzba_split_reshape_cat(qkvz, ba, 2, 4, 4, 2)
    assert qkv.dtype == z.dtype == torch.bfloat16 and b.dtype == a.dtype == torch.float16
