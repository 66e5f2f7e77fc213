"""Pins for oracle/conv1d.py (CPU only).

The v2 pin restates the reference's C++ golden loop
(triton_causal_conv1d_update_v2_test.cpp:138-223) element by element in
float64 numpy: an explicit per-channel, per-token recurrence, independent of
the oracle's per-sequence F.conv1d formulation.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import conv1d as oc


def golden_v2_loop(x, state, w, bias, qsl, mql, slots=None, init=None,
                   last=None, pad=-1, activation=True):
    """Literal per-element loop of causal_conv1d_update_ref_v2 (float64)."""
    x = x.astype(np.float64)
    st = state.astype(np.float64).copy()
    w = w.astype(np.float64)
    bias = np.zeros(w.shape[0]) if bias is None else bias.astype(np.float64)
    lines, D, S = st.shape
    W = w.shape[1]
    out = np.zeros_like(x)

    def res(b, col):
        if slots is None:
            return b
        return int(slots[b]) if slots.ndim == 1 else int(slots[b, col])

    for b in range(len(qsl) - 1):
        start, end = qsl[b], qsl[b + 1]
        ln = end - start
        if ln <= 0:
            continue
        run = (W - 1) - (mql - ln)
        in_idx = res(b, 0 if init is None else init[b])
        if in_idx == pad:
            continue
        out_idx = res(b, 0 if last is None else last[b])
        in_ok = 0 <= in_idx < lines
        out_ok = 0 <= out_idx < lines
        keep_shift = run - ln if ln < run else 0
        tail = ln - run if ln >= run else 0
        for f in range(D):
            cols = [st[in_idx, f, k] if in_ok else 0.0 for k in range(W - 1)]
            for t in range(ln):
                xv = x[start + t, f]
                acc = bias[f]
                for k in range(W - 1):
                    acc += cols[k] * w[f, k]
                acc += xv * w[f, W - 1]
                out[start + t, f] = acc
                cols = cols[1:] + [xv] if W > 1 else cols
            if not out_ok or run <= 0:
                continue
            if ln < run:
                if in_ok:
                    for d in range(keep_shift):
                        st[out_idx, f, d] = st[in_idx, f, d + ln]
                for xt in range(ln):
                    if keep_shift + xt < run:
                        st[out_idx, f, keep_shift + xt] = x[start + xt, f]
            else:
                for d in range(run):
                    st[out_idx, f, d] = x[start + tail + d, f]
    if activation:
        out = out / (1.0 + np.exp(-out))
    return out, st


@pytest.mark.parametrize("case", ["apc_decode", "pad_width5", "prefill_varlen"])
def test_v2_oracle_matches_golden_loop(case):
    g = torch.Generator().manual_seed(0)
    D = 24
    if case == "apc_decode":  # triton_causal_conv1d_update_v2_test.cpp:238-315
        W, B = 4, 4
        x = torch.randn(B, D, generator=g, dtype=torch.float64)
        state = torch.randn(2 * B, D, W - 1, generator=g, dtype=torch.float64)
        slots = torch.stack([torch.arange(B), torch.arange(B) + B], 1).int()
        last = torch.ones(B, dtype=torch.int32)
        init = torch.zeros(B, dtype=torch.int32)
        qsl = torch.arange(B + 1, dtype=torch.int32)
        mql, pad = 1, -1
    elif case == "pad_width5":  # :372-446
        W = 5
        x = torch.randn(5, D, generator=g, dtype=torch.float64)
        state = torch.randn(4, D, W - 1, generator=g, dtype=torch.float64)
        slots = torch.tensor([[0, 1], [-7, -7], [2, 3]], dtype=torch.int32)
        last = torch.tensor([1, 0, 1], dtype=torch.int32)
        init = torch.zeros(3, dtype=torch.int32)
        qsl = torch.tensor([0, 3, 3, 5], dtype=torch.int32)
        mql, pad = 3, -7
    else:
        W = 4
        qsl = torch.tensor([0, 5, 6, 13, 13, 20], dtype=torch.int32)
        x = torch.randn(20, D, generator=g, dtype=torch.float64)
        state = torch.randn(5, D, W - 1, generator=g, dtype=torch.float64)
        slots, last, init = torch.tensor([4, 0, 2, 1, 3], dtype=torch.int32), None, None
        mql, pad = 7, -1
    w = torch.randn(D, W, generator=g, dtype=torch.float64)
    bias = torch.randn(D, generator=g, dtype=torch.float64)
    out, st = oc.causal_conv1d_update_v2(
        x, state, w, bias, True, slots, qsl, mql, pad, last, init,
        dtype=torch.float64)
    ref_out, ref_st = golden_v2_loop(
        x.numpy(), state.numpy(), w.numpy(), bias.numpy(), qsl.tolist(), mql,
        None if slots is None else slots.numpy(),
        None if init is None else init.numpy(),
        None if last is None else last.numpy(), pad)
    # rows of pad sequences are unspecified in the reference; none here write
    np.testing.assert_allclose(out.numpy(), ref_out, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(st.numpy(), ref_st, rtol=0, atol=0)


def test_update_identity_weight_and_state_shift():
    # weight e_{W-1}: out = silu(x); state shifts left by seqlen.
    g = torch.Generator().manual_seed(1)
    B, D, T, W, S = 3, 16, 2, 4, 5
    x = torch.randn(B, D, T, generator=g, dtype=torch.float64)
    state = torch.randn(B, D, S, generator=g, dtype=torch.float64)
    w = torch.zeros(D, W, dtype=torch.float64)
    w[:, -1] = 1
    out, st = oc.causal_conv1d_update(x, state, w, None, True, dtype=torch.float64)
    torch.testing.assert_close(out, F.silu(x))
    torch.testing.assert_close(st, torch.cat([state, x], -1)[..., -S:])


def test_update_first_tap_reads_oldest_window_element():
    # weight e_0 with S = W-1 and T = 1 picks state[..., 0].
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 8, generator=g, dtype=torch.float64)
    state = torch.randn(2, 8, 3, generator=g, dtype=torch.float64)
    w = torch.zeros(8, 4, dtype=torch.float64)
    w[:, 0] = 1
    out, _ = oc.causal_conv1d_update(x, state, w, None, False, dtype=torch.float64)
    torch.testing.assert_close(out, state[..., 0])


def test_update_skips_pad_slots():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 8, generator=g)
    state = torch.randn(3, 8, 3, generator=g)
    w = torch.randn(8, 4, generator=g)
    idx = torch.tensor([2, -1, 0], dtype=torch.int32)
    out, st = oc.causal_conv1d_update(x, state, w, None, True, idx, -1)
    assert torch.equal(st[1], state[1])
    assert torch.equal(out[1], torch.zeros(8))
    assert torch.equal(st[2, :, -1], x[0])


def test_v2_prefill_rule_keeps_last_inputs():
    g = torch.Generator().manual_seed(4)
    qsl = torch.tensor([0, 5, 7], dtype=torch.int32)
    x = torch.randn(7, 6, generator=g)
    state = torch.zeros(2, 6, 3)
    w = torch.randn(6, 4, generator=g)
    _, st_ref = oc.causal_conv1d_update_v2(x, state, w, None, True, None, qsl, 5)
    _, st_pre = oc.causal_conv1d_update_v2(x, state, w, None, True, None, qsl, 5,
                                           state_rule=1)
    # reference rule: the shorter sequence (len 2) gets run = 3 - 3 = 0
    assert torch.equal(st_ref[1], torch.zeros(6, 3))
    assert torch.equal(st_pre[1][:, 1:], x[5:7].t()) and torch.equal(st_pre[1][:, 0], torch.zeros(6))
    assert torch.equal(st_pre[0], x[2:5].t())


def golden_v2_spec_loop(x, state, w, bias, qsl, mql, acc, slots=None,
                        activation=True):
    """Per-element float64 restatement of the speculative-decoding branch of
    causal_conv1d_update_ref_v2 (test_causal_conv1d_update_v2.py:290-335):
    eff = W-1 + mql-1; run = eff - (mql - len); the window starts at column
    off = accepted-1 of the input slot; when len < run the new state is
    old[off+1 : off+1+keep] (keep = run - len) followed by the inputs, else
    the last `run` inputs.  Indexing is written out column by column, with
    no slicing shared with oracle/conv1d.py."""
    x = x.astype(np.float64)
    st = state.astype(np.float64).copy()
    old = st.copy()
    w = w.astype(np.float64)
    bias = np.zeros(w.shape[0]) if bias is None else bias.astype(np.float64)
    lines, D, S = st.shape
    W = w.shape[1]
    eff = (W - 1) + (mql - 1)
    out = np.zeros_like(x)
    for b in range(len(qsl) - 1):
        start, end = qsl[b], qsl[b + 1]
        ln = end - start
        if ln <= 0:
            continue
        slot = b if slots is None else int(slots[b])
        off = int(acc[b]) - 1
        run = eff - (mql - ln)
        assert run >= 1 and off >= 0 and off + W - 1 <= S
        for f in range(D):
            for t in range(ln):
                acc_v = bias[f]
                for j in range(W):
                    # window position j of output t: history column off+t+j
                    # while t+j < W-1, else input token t+j-(W-1)
                    p = t + j
                    if p < W - 1:
                        val = old[slot, f, off + p]
                    else:
                        val = x[start + p - (W - 1), f]
                    acc_v += w[f, j] * val
                out[start + t, f] = acc_v
            if ln >= run:
                for d in range(run):
                    st[slot, f, d] = x[start + ln - run + d, f]
            else:
                keep = run - ln
                assert off + 1 + keep <= S  # the reference raises otherwise
                for d in range(keep):
                    st[slot, f, d] = old[slot, f, off + 1 + d]
                for t in range(ln):
                    st[slot, f, keep + t] = x[start + t, f]
    if activation:
        out = out / (1.0 + np.exp(-out))
    return out, st


def _spec_case(seed, W, lens, varlen=True):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    mql = max(lens)
    S = (W - 1) + (mql - 1)
    D = 12
    qsl = [0]
    for n in lens:
        qsl.append(qsl[-1] + n)
    x = torch.randn(qsl[-1], D, generator=g, dtype=torch.float64)
    state = torch.randn(B + 1, D, S, generator=g, dtype=torch.float64)
    w = torch.randn(D, W, generator=g, dtype=torch.float64)
    bias = torch.randn(D, generator=g, dtype=torch.float64)
    slots = torch.randperm(B + 1, generator=g)[:B].int()
    acc = torch.tensor([1 + int(torch.randint(0, mql, (1,), generator=g)) for _ in lens],
                       dtype=torch.int32)
    return x, state, w, bias, torch.tensor(qsl, dtype=torch.int32), mql, acc, slots


@pytest.mark.parametrize("W", [2, 3, 4, 5])
@pytest.mark.parametrize("lens", [[3, 3, 3], [1, 4, 2, 4], [2, 1]])
def test_v2_spec_oracle_matches_per_element_loop(W, lens):
    x, state, w, bias, qsl, mql, acc, slots = _spec_case(10 * W + len(lens), W, lens)
    out, st = oc.causal_conv1d_update_v2(
        x, state, w, bias, True, slots, qsl, mql, num_accepted_tokens=acc,
        dtype=torch.float64)
    ref_out, ref_st = golden_v2_spec_loop(
        x.numpy(), state.numpy(), w.numpy(), bias.numpy(), qsl.tolist(), mql,
        acc.numpy(), slots.numpy())
    np.testing.assert_allclose(out.numpy(), ref_out, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(st.numpy(), ref_st)


@pytest.mark.parametrize("W", [3, 4, 6])
def test_v2_spec_identity_weight_closed_form(W):
    # Weight e_{W-1}: out = silu(x) whatever the history; the new state is
    # old[off+1 : off+1+keep] (keep = W-2 for every length) followed by the
    # sequence's inputs; columns past run keep their old values.
    lens = [3, 1, 2]
    x, state, _, _, qsl, mql, acc, slots = _spec_case(W, W, lens)
    D = x.shape[1]
    w = torch.zeros(D, W, dtype=torch.float64)
    w[:, -1] = 1
    out, st = oc.causal_conv1d_update_v2(
        x, state, w, None, True, slots, qsl, mql, num_accepted_tokens=acc,
        dtype=torch.float64)
    torch.testing.assert_close(out, F.silu(x), rtol=1e-15, atol=1e-15)
    keep = W - 2
    for b, n in enumerate(lens):
        s, off = int(slots[b]), int(acc[b]) - 1
        start = int(qsl[b])
        expect = torch.cat([state[s, :, off + 1:off + 1 + keep], x[start:start + n].t()], 1)
        assert torch.equal(st[s, :, :keep + n], expect)
        assert torch.equal(st[s, :, keep + n:], state[s, :, keep + n:])
    untouched = sorted(set(range(state.shape[0])) - set(slots.tolist()))
    for s in untouched:
        assert torch.equal(st[s], state[s])


def test_v2_spec_first_tap_reads_accepted_column():
    # Weight e_0, one token per sequence: the output is the state column
    # off = accepted-1 (the oldest element of the window), pre-SiLU.
    W, lens = 4, [1, 1, 1]
    x, state, _, _, qsl, mql, _, slots = _spec_case(5, W, lens)
    mql = 3  # state holds W-1 + mql-1 = 5 columns; accepted 1..3
    state = torch.randn(4, x.shape[1], W - 1 + mql - 1, dtype=torch.float64)
    acc = torch.tensor([1, 2, 3], dtype=torch.int32)
    w = torch.zeros(x.shape[1], W, dtype=torch.float64)
    w[:, 0] = 1
    out, _ = oc.causal_conv1d_update_v2(
        x, state, w, None, False, slots, qsl, mql, num_accepted_tokens=acc,
        dtype=torch.float64)
    for b in range(3):
        assert torch.equal(out[b], state[int(slots[b]), :, int(acc[b]) - 1])
