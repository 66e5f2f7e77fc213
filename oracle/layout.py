"""CPU restatement of the GDN projection split (test infrastructure).

fused_qkvzba_split_reshape_cat: fused_qkvzba_split_reshape_cat_ref of
  triton_npu/triton_src/test_fused_qkvzba_split_reshape.py:463-506: rows of
  mixed_qkvz viewed as [num_heads_qk, q | k | v | z] and rows of mixed_ba
  as [num_heads_qk, b | a], re-concatenated head-major into mixed_qkv =
  [q | k | v], z [rows, num_heads_v, head_v], b and a [rows, num_heads_v].

Pins (tests/test_oracle_layout.py): the op is a permutation, so with an
index-valued input every output element names its source; those sources
are checked against positions worked out by hand for a small case, the
outputs are checked to be a bijection onto the input, and a literal
element-by-element loop restating the group layout reproduces them.
"""
from __future__ import annotations

import torch


def fused_qkvzba_split_reshape_cat(mixed_qkvz, mixed_ba, num_heads_qk: int, num_heads_v: int,
                                   head_qk: int, head_v: int):
    """(mixed_qkv, z, b, a) in the input dtypes."""
    rows = mixed_qkvz.shape[0]
    R = num_heads_v // num_heads_qk
    dt = head_qk * 2 + R * head_v * 2
    qkvz = mixed_qkvz.reshape(rows, num_heads_qk, dt)
    ba = mixed_ba.reshape(rows, num_heads_qk, 2 * R)
    q = qkvz[..., :head_qk]
    k = qkvz[..., head_qk:2 * head_qk]
    v = qkvz[..., 2 * head_qk:2 * head_qk + R * head_v]
    z = qkvz[..., 2 * head_qk + R * head_v:]
    mixed_qkv = torch.cat([q.reshape(rows, num_heads_qk * head_qk),
                           k.reshape(rows, num_heads_qk * head_qk),
                           v.reshape(rows, num_heads_v * head_v)], dim=-1)
    return (mixed_qkv.contiguous(), z.reshape(rows, num_heads_v, head_v).contiguous(),
            ba[..., :R].reshape(rows, num_heads_v).contiguous(),
            ba[..., R:].reshape(rows, num_heads_v).contiguous())


def source_of(num_heads_qk: int, num_heads_v: int, head_qk: int, head_v: int):
    """Element-by-element restatement of the group layout: for every output
    position, the index of its source element in a mixed_qkvz row (for
    mixed_qkv and z) or in a mixed_ba row (for b and a)."""
    R = num_heads_v // num_heads_qk
    dt = head_qk * 2 + R * head_v * 2
    src_qkv, src_z, src_b, src_a = [], [], [], []
    for part in range(2):  # all q, then all k
        for g in range(num_heads_qk):
            for e in range(head_qk):
                src_qkv.append(g * dt + part * head_qk + e)
    for hv in range(num_heads_v):  # v heads in order: group hv // R, slot hv % R
        g, j = divmod(hv, R)
        for e in range(head_v):
            src_qkv.append(g * dt + 2 * head_qk + j * head_v + e)
            src_z.append(g * dt + 2 * head_qk + R * head_v + j * head_v + e)
        src_b.append(g * 2 * R + j)
        src_a.append(g * 2 * R + R + j)
    return src_qkv, src_z, src_b, src_a
