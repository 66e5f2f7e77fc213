"""CPU restatements of the causal conv1d references (test infrastructure).

causal_conv1d_update: causal_conv1d_update_ref of
  triton_npu/triton_src/test_causal_conv1d_update.py:1158-1210 and
  triton_npu/test/triton_causal_conv1d_update_test.cpp:41-128 (no
  cache_seqlens): x_new = cat(state, x); state <- last state_len of x_new;
  out = F.conv1d(x_new, w, b, groups=dim)[..., -seqlen:], then SiLU.  The
  slot of batch row b is conv_state_indices[b] (pad_slot_id rows skipped),
  as the kernel test_causal_conv1d_update.py:886-939 indexes it.
causal_conv1d_update_v2: causal_conv1d_update_ref_v2 of
  triton_npu/test/triton_causal_conv1d_update_v2_test.cpp:59-229 (the
  authoritative final-state rule), extended with the speculative-decoding
  offsets of triton_npu/triton_src/test_causal_conv1d_update_v2.py:260-339
  (history at accepted-1, shift 1).  Outputs use a per-sequence F.conv1d
  over cat(history, x_s) in fp32.

All arithmetic is fp32 (or `dtype`); results keep fp32.  Pins
(tests/test_oracle_conv1d.py): a literal per-element restatement of the C++
golden loop in float64, identity/shift weights, and the state-rule cases of
the reference's gtests.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F


def _act(y, activation):
    return F.silu(y) if activation else y


def causal_conv1d_update(x: torch.Tensor, conv_state: torch.Tensor,
                         weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
                         activation: bool = True,
                         conv_state_indices: Optional[torch.Tensor] = None,
                         pad_slot_id: int = -1, dtype=torch.float32):
    """Returns (out [B, D(, T)], new conv_state); conv_state is not modified."""
    unsq = x.dim() == 2
    xs = x.unsqueeze(-1) if unsq else x
    B, D, T = xs.shape
    W = weight.shape[1]
    S = conv_state.shape[2]
    state = conv_state.to(dtype).clone()
    out = torch.zeros(B, D, T, dtype=dtype)
    w = weight.to(dtype).unsqueeze(1)
    b = bias.to(dtype) if bias is not None else None
    for i in range(B):
        slot = int(conv_state_indices[i]) if conv_state_indices is not None else i
        if conv_state_indices is not None and slot == pad_slot_id:
            continue
        x_new = torch.cat([state[slot], xs[i].to(dtype)], -1)  # [D, S+T]
        y = F.conv1d(x_new.unsqueeze(0), w, b, groups=D)[0, :, -T:]
        out[i] = _act(y, activation)
        state[slot] = x_new[:, -S:]
    return (out.squeeze(-1) if unsq else out), state


def _slot(slots, b, col):
    if slots is None:
        return b
    if slots.dim() == 1:
        return int(slots[b])
    return int(slots[b, col])


def causal_conv1d_update_v2(x: torch.Tensor, conv_state: torch.Tensor,
                            weight: torch.Tensor,
                            bias: Optional[torch.Tensor] = None,
                            activation: bool = True,
                            conv_state_indices: Optional[torch.Tensor] = None,
                            query_start_loc: Optional[torch.Tensor] = None,
                            max_query_len: int = -1, pad_slot_id: int = -1,
                            block_idx_last_scheduled_token: Optional[torch.Tensor] = None,
                            initial_state_idx: Optional[torch.Tensor] = None,
                            num_accepted_tokens: Optional[torch.Tensor] = None,
                            state_rule: int = 0, dtype=torch.float32):
    """Returns (out like x, new conv_state).  Rows of skipped (pad) sequences
    are left as zeros in `out`; conv_state is not modified in place."""
    if query_start_loc is None:
        xw = x.unsqueeze(-1) if x.dim() == 2 else x
        Bn, D, Tn = xw.shape
        xt = xw.transpose(1, 2).reshape(Bn * Tn, D)
        qsl = [i * Tn for i in range(Bn + 1)]
        seqlen = Tn
    else:
        xt = x
        D = x.shape[1]
        qsl = [int(v) for v in query_start_loc]
        Bn = len(qsl) - 1
        seqlen = max_query_len
    W = weight.shape[1]
    lines, _, S = conv_state.shape
    eff = W - 1 + (seqlen - 1 if num_accepted_tokens is not None else 0)
    state = conv_state.to(dtype).clone()
    old = conv_state.to(dtype).clone()
    out = torch.zeros(xt.shape[0], D, dtype=dtype)
    w = weight.to(dtype).unsqueeze(1)
    b = bias.to(dtype) if bias is not None else None
    pending = []
    for s in range(Bn):
        start, end = qsl[s], qsl[s + 1]
        ln = end - start
        if ln <= 0:
            continue
        init = int(initial_state_idx[s]) if initial_state_idx is not None else 0
        last = int(block_idx_last_scheduled_token[s]) if block_idx_last_scheduled_token is not None else 0
        in_idx = _slot(conv_state_indices, s, init)
        if conv_state_indices is not None and in_idx == pad_slot_id:
            continue
        out_idx = _slot(conv_state_indices, s, last)
        in_ok = 0 <= in_idx < lines
        out_ok = 0 <= out_idx < lines
        off = int(num_accepted_tokens[s]) - 1 if num_accepted_tokens is not None else 0
        hist = torch.zeros(D, W - 1, dtype=dtype)
        if in_ok and off >= 0 and off + W - 1 <= S:
            hist = old[in_idx, :, off:off + W - 1]
        seq = xt[start:end].to(dtype).t()  # [D, len]
        y = F.conv1d(torch.cat([hist, seq], -1).unsqueeze(0), w, b, groups=D)[0]
        out[start:end] = _act(y, activation).t()
        run = eff - (seqlen - ln) if state_rule == 0 else eff
        if not out_ok or run <= 0 or run > S:
            continue
        if ln >= run:
            new = seq[:, ln - run:]
            pending.append((out_idx, 0, new))
        else:
            keep = run - ln
            shift = 1 if num_accepted_tokens is not None else ln
            if in_ok and off >= 0:
                n = max(0, min(keep, S - off - shift))
                pending.append((out_idx, 0, old[in_idx, :, off + shift:off + shift + n]))
            pending.append((out_idx, keep, seq))
    for slot, pos, vals in pending:
        state[slot, :, pos:pos + vals.shape[1]] = vals
    if query_start_loc is None:
        o = out.reshape(Bn, seqlen, D).transpose(1, 2)
        if x.dim() == 2:
            o = o.squeeze(-1)
        return o, state
    return out, state
