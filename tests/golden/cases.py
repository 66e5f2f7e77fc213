"""Golden-vector cases, one or two per op family: seeded inputs, the CPU
oracle's outputs, and the GPU call of the same op (test infrastructure).

make_golden.py writes every case's inputs and oracle outputs to
golden_vectors.safetensors; tests/test_golden.py checks that the oracle
still reproduces them (CPU) and that the HIP kernels match them at the
parity tolerances (GPU).  The reference holds no golden vectors of its own
for this path, so these anchor the oracle as it stands, cross-checked by
the closed-form pins in tests/test_oracle_*.py.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

BF16 = dict(rtol=1.6e-2, atol=1e-2)   # bf16 outputs against fp32 references
STAT = dict(rtol=1e-4, atol=1e-5)     # fp32 norm statistics
F32 = dict(rtol=1e-4, atol=1e-4)      # fp32 outputs of fp32 math
STATE = dict(rtol=1e-3, atol_per_rms=1e-3, atol_max=1e-4)  # fp32 GDN states: atol = min(1e-4, 1e-3 * RMS(reference))
EXACT = dict(rtol=0.0, atol=0.0)      # permutations, state shifts

CASES = {}


def case(name):
    def reg(c):
        CASES[name] = c()
        return c
    return reg


def _bf(shape, g, scale=1.0, shift=0.0):
    return (torch.randn(*shape, generator=g) * scale + shift).to(torch.bfloat16)


@case("layer_norm_gated")
class LayerNormGated:
    """layer_norm_fwd: grouped LayerNorm (group 256) with bias and the
    z * sigmoid(z) gate after the norm."""
    tol = dict(y=BF16, mean=STAT, rstd=STAT)

    def inputs(self, g):
        return dict(x=_bf((16, 512), g), w=_bf((512,), g, 0.1, 1.0), b=_bf((512,), g, 0.1),
                    z=_bf((16, 512), g))

    def oracle(self, t):
        from oracle import norm as on
        y, mean, rstd = on.layer_norm_fwd(t["x"], t["w"], t["b"], 1e-5, z=t["z"], group_size=256,
                                          norm_before_gate=True, is_rms_norm=False)
        return dict(y=y, mean=mean, rstd=rstd)

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        y, mean, rstd = ops.layer_norm_fwd(t["x"], t["w"], t["b"], 1e-5, t["z"], 256, True, False,
                                           return_stats=True)
        return dict(y=y, mean=mean, rstd=rstd)


@case("rms_norm_gate_first")
class RmsGateFirst:
    """layer_norm_fwd: RMSNorm over groups of 128, no bias, gate before the
    statistics (norm_before_gate = false)."""
    tol = dict(y=BF16, rstd=STAT)

    def inputs(self, g):
        return dict(x=_bf((16, 512), g), w=_bf((512,), g, 0.1, 1.0), z=_bf((16, 512), g))

    def oracle(self, t):
        from oracle import norm as on
        y, _, rstd = on.layer_norm_fwd(t["x"], t["w"], None, 1e-6, z=t["z"], group_size=128,
                                       norm_before_gate=False, is_rms_norm=True)
        return dict(y=y, rstd=rstd)

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        y, _, rstd = ops.layer_norm_fwd(t["x"], t["w"], None, 1e-6, t["z"], 128, False, True,
                                        return_stats=True)
        return dict(y=y, rstd=rstd)


@case("gemma_rms_norm")
class Gemma:
    tol = dict(y=BF16, rstd=STAT)

    def inputs(self, g):
        return dict(x=_bf((16, 512), g), gamma=_bf((512,), g, 0.1))

    def oracle(self, t):
        from oracle import norm as on
        y, rstd = on.gemma_rms_norm(t["x"], t["gamma"], 1e-5)
        return dict(y=y, rstd=rstd)

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        y, rstd = ops.npu_gemma_rms_norm(t["x"], t["gamma"], 1e-5)
        return dict(y=y, rstd=rstd.reshape(-1))


@case("l2norm_last_dim")
class L2Norm:
    tol = dict(y=BF16)

    def inputs(self, g):
        return dict(x=_bf((32, 128), g))

    def oracle(self, t):
        from oracle import norm as on
        return dict(y=on.l2norm_last_dim(t["x"]))

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        return dict(y=ops.npu_l2norm_last_dim(t["x"]))


@case("split_rmsnorm_rope")
class SplitRope:
    """fp32 q/k RMSNorm + neox RoPE, 4 q and 2 kv heads of 64, sin / cos rows
    from positions (theta 1e6)."""
    tol = dict(q=F32, k=F32, v=EXACT)

    def inputs(self, g):
        from oracle import rope as orp
        pos = torch.randint(0, 4096, (8,), generator=g)
        cos, sin = orp.neox_cos_sin(pos, orp.inv_freq_table(64, 1e6))
        return dict(qkv=torch.randn(8, 512, generator=g), sin=sin, cos=cos,
                    qw=torch.randn(64, generator=g) * 0.1 + 1, kw=torch.randn(64, generator=g) * 0.1 + 1)

    def oracle(self, t):
        from oracle import rope as orp
        q, k, v = orp.split_rmsnorm_rope(t["qkv"], t["sin"], t["cos"], t["qw"], t["kw"], 256, 128, 64,
                                         1e-6)
        return dict(q=q, k=k, v=v)

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        q, k, v = ops.npu_split_rmsnorm_rope(t["qkv"], t["sin"], t["cos"], t["qw"], t["kw"], 256, 128,
                                             64, 1e-6)
        return dict(q=q, k=k, v=v)


@case("rope_inplace")
class RopeInplace:
    tol = dict(x=BF16)

    def inputs(self, g):
        return dict(x=_bf((8, 4, 128), g), sin=_bf((8, 64), g), cos=_bf((8, 64), g))

    def oracle(self, t):
        from oracle import rope as orp
        return dict(x=orp.rope_inplace_ref(t["x"], t["sin"], t["cos"], 64).float())

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        x = t["x"].clone()
        ops.rope_inplace(x, t["sin"], t["cos"], 64)
        return dict(x=x)


@case("conv1d_update")
class ConvUpdate:
    """Single-token conv update, width 4, SiLU, state slots out of order."""
    tol = dict(y=BF16, state=EXACT)

    def inputs(self, g):
        return dict(x=_bf((4, 64), g), state=_bf((6, 64, 3), g), w=_bf((64, 4), g, 0.5),
                    idx=torch.tensor([2, 0, 5, 3], dtype=torch.int32))

    def oracle(self, t):
        from oracle import conv1d as oc
        y, st = oc.causal_conv1d_update(t["x"], t["state"], t["w"], None, True, t["idx"])
        return dict(y=y.float(), state=st.to(torch.bfloat16))

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        st = t["state"].clone()
        y = ops.npu_causal_conv1d_update(t["x"], st, t["w"], True, conv_state_indices=t["idx"])
        return dict(y=y, state=st)


@case("conv1d_varlen")
class ConvVarlen:
    """Varlen conv (npu_causal_conv1d_update_v2), 3 sequences, non-zero
    initial states and the reference's final-state rule."""
    tol = dict(y=BF16, state=EXACT)

    def inputs(self, g):
        return dict(x=_bf((50, 64), g), state=_bf((3, 64, 3), g), w=_bf((64, 4), g, 0.5),
                    qsl=torch.tensor([0, 7, 30, 50], dtype=torch.int32))

    def oracle(self, t):
        from oracle import conv1d as oc
        y, st = oc.causal_conv1d_update_v2(t["x"], t["state"].clone(), t["w"], None, True, None,
                                           t["qsl"], 23)
        return dict(y=y.float(), state=st.to(torch.bfloat16))

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        st = t["state"].clone()
        y = ops.npu_causal_conv1d_update_v2(t["x"], st, t["w"], True, query_start_loc=t["qsl"],
                                            max_query_len=23)
        return dict(y=y, state=st)


@case("gdn_recurrent")
class GdnRecurrent:
    """Recurrent gated delta rule, 3 sequences x 1 token, 2 qk / 4 v heads,
    head dims 64, in-kernel l2norm, states updated in place."""
    tol = dict(o=BF16, state=STATE)

    def inputs(self, g):
        return dict(q=_bf((3, 2, 64), g), k=_bf((3, 2, 64), g), v=_bf((3, 4, 64), g),
                    gate=F.logsigmoid(torch.randn(3, 4, generator=g)),
                    beta=torch.sigmoid(torch.randn(3, 4, generator=g)).bfloat16(),
                    h0=torch.randn(3, 4, 64, 64, generator=g) * 0.1,
                    cu=torch.arange(4, dtype=torch.int32), idx=torch.arange(3, dtype=torch.int32))

    def oracle(self, t):
        from oracle import gdn as og
        o, st = og.recurrent_gdn(t["q"], t["k"], t["v"], t["gate"], t["beta"], 0.125, t["h0"],
                                 t["cu"], t["idx"])
        return dict(o=o.float(), state=st.float())

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        st = t["h0"].clone()
        o, _ = ops.npu_fused_recurrent_gated_delta_rule(
            t["q"][None], t["k"][None], t["v"][None], t["gate"][None], t["beta"][None], 0.125, st,
            True, t["cu"], t["idx"])
        return dict(o=o[0], state=st)


@case("gdn_chunk")
class GdnChunk:
    """Chunked gated delta rule, 2 sequences (50 and 100 tokens), 1 qk / 2 v
    heads of 128, in-op l2norm, initial and final states."""
    tol = dict(o=BF16, state=STATE)

    def inputs(self, g):
        return dict(q=_bf((1, 150, 1, 128), g), k=_bf((1, 150, 1, 128), g), v=_bf((1, 150, 2, 128), g),
                    gate=F.logsigmoid(torch.randn(1, 150, 2, generator=g)),
                    beta=torch.sigmoid(torch.randn(1, 150, 2, generator=g)).bfloat16(),
                    h0=torch.randn(2, 2, 128, 128, generator=g) * 0.1,
                    cu=torch.tensor([0, 50, 150], dtype=torch.int32))

    def oracle(self, t):
        from oracle import gdn as og
        o, st = og.chunk_gdn(t["q"], t["k"], t["v"], t["gate"], t["beta"], None, t["h0"], t["cu"],
                             use_qk_l2norm=True)
        return dict(o=o, state=st)

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        o, st = ops.npu_chunk_gated_delta_rule(t["q"], t["k"], t["v"], t["gate"], t["beta"], None,
                                               t["h0"], True, t["cu"], False, True)
        return dict(o=o, state=st)


@case("gdn_gating")
class Gating:
    tol = dict(g=dict(rtol=1e-3, atol=1e-3), beta=BF16)

    def inputs(self, g):
        return dict(A_log=torch.randn(4, generator=g), a=_bf((16, 4), g), b=_bf((16, 4), g),
                    dt_bias=torch.randn(4, generator=g))

    def oracle(self, t):
        from oracle import gating as ogt
        gg, bb = ogt.fused_gdn_gating(t["A_log"], t["a"], t["b"], t["dt_bias"])
        return dict(g=gg, beta=bb.float())

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        gg, bb = ops.npu_fused_gdn_gating(t["A_log"], t["a"], t["b"], t["dt_bias"])
        return dict(g=gg, beta=bb)


@case("qkvzba_split")
class QkvzbaSplit:
    """Projection split, 2 qk heads / 4 v heads (2 per group), head dims 32."""
    tol = dict(mixed_qkv=EXACT, z=EXACT, b=EXACT, a=EXACT)

    def inputs(self, g):
        return dict(qkvz=_bf((8, 2 * (2 * 32 + 2 * 2 * 32)), g), ba=_bf((8, 2 * 4), g))

    def oracle(self, t):
        from oracle import layout as ol
        qkv, z, b, a = ol.fused_qkvzba_split_reshape_cat(t["qkvz"], t["ba"], 2, 4, 32, 32)
        return dict(mixed_qkv=qkv, z=z, b=b, a=a)

    def gpu(self, t):
        from torch_npu_ops_amd import ops
        qkv, z, b, a = ops.npu_fused_qkvzba_split_reshape_cat(t["qkvz"], t["ba"], 2, 4, 32, 32)
        return dict(mixed_qkv=qkv, z=z, b=b, a=a)


@case("gdn_stages")
class GdnStages:
    """The chunked pipeline stage by stage (cumsum, K K^T, solve_tril,
    recompute_w_u, fwd_h, fwd_o), 3 sequences (1, 64 and 85 tokens), 1 qk /
    2 v heads of 128.  Each stage's inputs are the oracle's outputs of the
    stages before it (stored), so every stage kernel is checked on its own."""
    tol = dict(gc=dict(rtol=1e-5, atol=1e-5), A=F32, Ai=dict(rtol=1e-3, atol=1e-3), w=BF16, u=BF16, h=BF16, vnew=BF16,
               ht=STATE, o=BF16)

    def inputs(self, g):
        return dict(q=_bf((150, 1, 128), g), k=_bf((150, 1, 128), g), v=_bf((150, 2, 128), g),
                    gate=F.logsigmoid(torch.randn(150, 2, generator=g)),
                    beta=torch.sigmoid(torch.randn(150, 2, generator=g)).bfloat16(),
                    h0=torch.randn(3, 2, 128, 128, generator=g) * 0.1,
                    cu=torch.tensor([0, 1, 65, 150], dtype=torch.int32))

    def oracle(self, t):
        from oracle import gdn as og
        k = og.l2norm(t["k"].float()).bfloat16()
        q = og.l2norm(t["q"].float()).bfloat16()
        cu = t["cu"]
        gc = og.chunk_local_cumsum(t["gate"].unsqueeze(0), cu)[0]
        A = og.chunk_scaled_dot_kkt(k, t["beta"], gc, cu)
        Ai = og.solve_tril(A, cu)
        w, u = og.recompute_w_u(k, t["v"], t["beta"], gc, Ai, cu)
        w, u = w.bfloat16(), u.bfloat16()
        h, vnew, ht = og.chunk_fwd_h(k, w, u, gc, t["h0"], cu)
        o = og.chunk_fwd_o(q, k, vnew.bfloat16(), h.bfloat16(), gc, 0.0883883, cu)
        # h and v_new are bf16 on the GPU side (the reference's stage dtypes)
        return dict(gc=gc, A=A, Ai=Ai, w=w.float(), u=u.float(), h=h.bfloat16(),
                    vnew=vnew.bfloat16(), ht=ht, o=o)

    def gpu_with_golden(self, t, out, dev):
        from torch_npu_ops_amd import ops
        from oracle import gdn as og

        def b(x):
            return x.unsqueeze(0).to(dev)
        k = og.l2norm(t["k"].float()).bfloat16()
        q = og.l2norm(t["q"].float()).bfloat16()
        cu = t["cu"].to(dev)
        got = {}
        got["gc"] = ops.npu_chunk_local_cumsum(b(t["gate"]), 64, cu)[0]
        got["A"] = ops.npu_chunk_scaled_dot_kkt_fwd(b(k), b(t["beta"]), b(out["gc"]), 64, cu)[0]
        got["Ai"] = ops.npu_solve_tril(b(out["A"]), 64, cu)[0]
        w, u = ops.npu_recompute_w_u_fwd(b(k), b(t["v"]), b(t["beta"]), b(out["gc"]),
                                         b(out["Ai"]), cu)
        got["w"], got["u"] = w[0], u[0]
        h, vnew, ht = ops.npu_chunk_gated_delta_rule_fwd_h(
            b(k), b(out["w"].bfloat16()), b(out["u"].bfloat16()), b(out["gc"]), t["h0"].to(dev),
            True, 64, True, cu)
        got["h"], got["vnew"], got["ht"] = h[0], vnew[0, :150], ht
        got["o"] = ops.npu_chunk_fwd_o(b(q), b(k), b(out["vnew"].bfloat16()),
                                       out["h"].bfloat16().unsqueeze(0).to(dev), b(out["gc"]),
                                       0.0883883, 64, cu)[0, :150]
        return got
