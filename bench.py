#!/usr/bin/env python3
"""Benchmark of the xLLM op set on one MI355X.

    python bench.py [--steps K] [--warmup W] [--op NAME] [--no-cpu] [--eager]

One step = one call of an op on its BASELINE config with inputs already
resident in HBM.  HIP events on the stream the kernels run on bracket the K
timed calls, launched back to back.  Ops that move >= 100 MB per call are
launched eagerly (the GPU queue stays ahead of the Python binding); the
smaller ops (configs 1 and 3b, and the gating / in-place RoPE lines), whose
kernels are not much longer than a Python launch, are captured in one HIP
graph that is replayed.  Inputs
rotate over several buffer sets whose total exceeds the 256 MB Infinity
Cache, so timings see HBM.  Before its W warm-up calls every op runs
untimed for SETTLE_S seconds, so that the GPU clocks have settled at their
sustained-load level when the timed calls start.

Rank 0 prints ONE JSON line:
  value        achieved GB/s of the headline op (algorithmic bytes / time)
  roofline     the headline kernel's achieved / peak
  cpu_baseline the oracle (CPU restatement of the reference) on host cores
  ops          every op's line (config, us per call, GB/s or tokens/s,
               roofline)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
MFMA_BF16_TFS = 2500.0  # dense bf16
ROTATE_BYTES = 1 << 30  # >= 1 GiB of distinct buffers per op
MAX_SETS = 128


def _cgroup_cpus():
    """CPUs granted by the cgroup v2 quota (cpu.max), or None if unlimited."""
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota == "max":
            return None
        return max(1, -(-int(quota) // int(period)))
    except (OSError, ValueError):
        return None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_threads():
    """Threads for the CPU baseline: every core this process may run on
    (os.cpu_count(), narrowed by the affinity mask and the cgroup quota when
    they grant fewer, so the baseline is not run oversubscribed)."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:
        pass
    q = _cgroup_cpus()
    return min(n, q) if q else n

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def _randn(shape, gen, dtype, scale=1.0, shift=0.0):
    return (torch.randn(shape, generator=gen) * scale + shift).to(dtype)


def _cur_stream():
    return torch.cuda.current_stream().cuda_stream


def _ok(st, lib):
    if st:
        from torch_npu_ops_amd import _lib
        raise RuntimeError(_lib.status_string(st))


class Case:
    """One BASELINE config.  sets(dev, n) returns n closures, each running
    the op once on its own buffers (stream read at call time); cpu()
    returns the CPU baseline closure, a description and the factor that
    scales one closure call to one full config call."""
    name = ""
    config = ""
    kernel = ""
    algo_bytes = 0
    timing = "eager"  # or "graph" for ops shorter than a Python launch
    source = ""  # the csrc/*.hip file of `kernel`

    def sets(self, dev, n):
        raise NotImplementedError

    def cpu(self):
        raise NotImplementedError


class LayerNormCase(Case):
    name = "layer_norm_fwd"
    config = ("config 2a: layer_norm_fwd bf16 x[16384,4096], group_size 4096, "
              "affine w~N(1,0.1) b~N(0,0.1), eps 1e-5, outputs y + fp32 mean/rstd")
    source = "norm.hip"
    kernel = "ln_tile_kernel<TPG=128,NV=4,z=0>"
    M, N = 16384, 4096
    # x + y (bf16) + mean/rstd (fp32) + w/b (bf16)
    algo_bytes = M * N * 2 * 2 + M * 4 * 2 + N * 2 * 2

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.x = _randn((self.M, self.N), g, torch.bfloat16)
        self.w = _randn((self.N,), g, torch.bfloat16, 0.1, 1.0)
        self.b = _randn((self.N,), g, torch.bfloat16, 0.1)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        w, b = self.w.to(dev), self.b.to(dev)
        out = []
        for _ in range(n):
            x = self.x.to(dev)
            y = torch.empty_like(x)
            mean = torch.empty(self.M, dtype=torch.float32, device=dev)
            rstd = torch.empty(self.M, dtype=torch.float32, device=dev)

            def run(x=x, y=y, mean=mean, rstd=rstd):
                _ok(lib.xk_layer_norm_fwd(
                    x.data_ptr(), self.N, y.data_ptr(), self.N, w.data_ptr(),
                    b.data_ptr(), None, 0, mean.data_ptr(), rstd.data_ptr(),
                    self.M, self.N, self.N, 1e-5, 1, 0, _lib.XK_BF16,
                    _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import norm as on
        x, w, b = self.x, self.w, self.b
        return (lambda: on.layer_norm_fwd(x, w, b, 1e-5),
                "full config 2a (16384x4096), fp32 math on bf16 input", 1.0)


class GemmaCase(Case):
    name = "gemma_rms_norm"
    config = ("config 2b: Gemma RMSNorm bf16 x[16384,4096], gamma~N(1,0.1) "
              "applied as (1+gamma), eps 1e-5, outputs y + fp32 rstd")
    source = "norm.hip"
    kernel = "ln_tile_kernel<TPG=128,NV=4,z=0>"
    M, N = 16384, 4096
    algo_bytes = M * N * 2 * 2 + M * 4 + N * 2

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.x = _randn((self.M, self.N), g, torch.bfloat16)
        self.gamma = _randn((self.N,), g, torch.bfloat16, 0.1, 1.0)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        gamma = self.gamma.to(dev)
        out = []
        for _ in range(n):
            x = self.x.to(dev)
            y = torch.empty_like(x)
            rstd = torch.empty(self.M, dtype=torch.float32, device=dev)

            def run(x=x, y=y, rstd=rstd):
                _ok(lib.xk_gemma_rms_norm(
                    x.data_ptr(), self.N, y.data_ptr(), self.N,
                    gamma.data_ptr(), rstd.data_ptr(), self.M, self.N, 1e-5,
                    _lib.XK_BF16, _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import norm as on
        x, gamma = self.x, self.gamma
        return (lambda: on.gemma_rms_norm(x, gamma, 1e-5),
                "full config 2b (16384x4096), fp32 math on bf16 input", 1.0)


class GatedRmsNormCase(Case):
    name = "gated_rms_norm"
    config = ("next row (layer_norm_fwd gated RMSNorm epilogue, the reference's nomask "
              "kernel shape): GDN output of the prefill config as rows of one head, "
              "x and z bf16 [524288, 128] (16384 tokens x 32 heads), group_size 128, "
              "RMS, gate z*sigmoid(z) after the norm, no bias, eps 1e-6; outputs y + "
              "fp32 rstd")
    source = "norm.hip"
    kernel = "ln_tile_kernel<TPG=8,NV=2,z=1>"
    M, N = 524288, 128
    # x, z, y (bf16) + rstd (fp32) + weight
    algo_bytes = M * N * 2 * 3 + M * 4 + N * 2

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.x = _randn((self.M, self.N), g, torch.bfloat16)
        self.z = _randn((self.M, self.N), g, torch.bfloat16)
        self.w = _randn((self.N,), g, torch.bfloat16, 0.1, 1.0)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        w = self.w.to(dev)
        out = []
        for _ in range(n):
            x, z = self.x.to(dev), self.z.to(dev)
            y = torch.empty_like(x)
            rstd = torch.empty(self.M, dtype=torch.float32, device=dev)

            def run(x=x, z=z, y=y, rstd=rstd):
                _ok(lib.xk_layer_norm_fwd(
                    x.data_ptr(), self.N, y.data_ptr(), self.N, w.data_ptr(), None,
                    z.data_ptr(), self.N, None, rstd.data_ptr(), self.M, self.N, self.N,
                    1e-6, 1, 1, _lib.XK_BF16, _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import norm as on
        x, z, w = self.x, self.z, self.w
        return (lambda: on.layer_norm_fwd(x, w, None, 1e-6, z=z, group_size=128,
                                          norm_before_gate=True, is_rms_norm=True),
                "full shape (524288 x 128), fp32 math on bf16 input", 1.0)


class RopeInplaceCase(Case):
    name = "rope_inplace"
    config = ("next row (rope_inplace, GPT-J interleaved partial RoPE): x bf16 "
              "[16384, 16, 512] rotated in place on its last 64 elements, sin / cos "
              "bf16 [16384, 64]")
    source = "rope.hip"
    kernel = "rope_inplace_tok_kernel"
    timing = "graph"
    T, H, HID, RD = 16384, 16, 512, 64
    # rope part of x read + written, sin / cos read (bf16)
    algo_bytes = T * H * RD * 2 * 2 + 2 * T * RD * 2
    # (rows, row bytes, rotated tail bytes) for the strided-pattern floor
    tail_floor = (T * H, HID * 2, RD * 2)

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.x = _randn((self.T, self.H, self.HID), g, torch.bfloat16)
        self.sin = _randn((self.T, self.RD), g, torch.bfloat16)
        self.cos = _randn((self.T, self.RD), g, torch.bfloat16)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        out = []
        for _ in range(n):
            x, sin, cos = self.x.to(dev), self.sin.to(dev), self.cos.to(dev)

            def run(x=x, sin=sin, cos=cos):
                _ok(lib.xk_rope_inplace(x.data_ptr(), self.T * self.H, self.H, self.HID,
                                        self.HID, sin.data_ptr(), cos.data_ptr(), self.RD,
                                        self.RD, _lib.XK_BF16, _lib.XK_BF16,
                                        _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import rope as orp
        a = (self.x, self.sin, self.cos, self.RD)
        return (lambda: orp.rope_inplace_ref(*a), "full shape, fp32 math", 1.0)


class RopeCase(Case):
    name = "split_rmsnorm_rope"
    config = ("config 1: split q/k RMSNorm + neox RoPE fp32, 256 tokens, 32 q + "
              "8 kv heads, head_dim 128, eps 1e-6, theta 1e6, sin/cos rows from "
              "positions U[0,4096)")
    source = "rope.hip"
    kernel = "split_rmsnorm_rope_kernel"
    timing = "graph"
    T, HQ, HKV, HD = 256, 32, 8, 128
    # qkv in + q/k/v out (fp32) + q/k weights + sin/cos rows
    algo_bytes = (T * (HQ + 2 * HKV) * HD * 4 * 2 + 2 * HD * 4 + 2 * T * HD * 4)

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        hid = (self.HQ + 2 * self.HKV) * self.HD
        self.qkv = _randn((self.T, hid), g, torch.float32)
        self.qw = _randn((self.HD,), g, torch.float32, 0.1, 1.0)
        self.kw = _randn((self.HD,), g, torch.float32, 0.1, 1.0)
        pos = torch.randint(0, 4096, (self.T,), generator=g)
        # neox rows: cos/sin of pos * theta^(-2i/HD), each half repeated.
        i = torch.arange(0, self.HD, 2, dtype=torch.float64)
        inv = (1.0 / (1e6 ** (i / self.HD))).to(torch.float32)
        f = pos.to(torch.float32)[:, None] * inv[None, :]
        self.cos = torch.cat([f.cos(), f.cos()], -1)
        self.sin = torch.cat([f.sin(), f.sin()], -1)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        qw, kw = self.qw.to(dev), self.kw.to(dev)
        qh, kvh = self.HQ * self.HD, self.HKV * self.HD
        out = []
        for _ in range(n):
            qkv, sin, cos = self.qkv.to(dev), self.sin.to(dev), self.cos.to(dev)
            q = torch.empty(self.T, qh, device=dev)
            k = torch.empty(self.T, kvh, device=dev)
            v = torch.empty(self.T, kvh, device=dev)

            def run(qkv=qkv, sin=sin, cos=cos, q=q, k=k, v=v):
                _ok(lib.xk_split_rmsnorm_rope(
                    qkv.data_ptr(), qkv.stride(0), self.T, sin.data_ptr(),
                    cos.data_ptr(), self.HD, None, _lib.XK_I64, None,
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), qw.data_ptr(), None,
                    kw.data_ptr(), None, _lib.XK_F32, qh, kvh, self.HD, 1e-6,
                    _lib.XK_F32, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import rope as orp
        a = (self.qkv, self.sin, self.cos, self.qw, self.kw,
             self.HQ * self.HD, self.HKV * self.HD, self.HD, 1e-6)
        return (lambda: orp.split_rmsnorm_rope(*a),
                "full config 1 (256 tokens), fp32", 1.0)


class RopePrefillCase(Case):
    """Config 1's op at a prefill size, with cos/sin computed in registers
    from positions: config 1 (256 tokens, 12.8 MB) is bounded by launch
    latency, this shows the same kernel where HBM is the bound."""
    name = "split_rmsnorm_rope_prefill"
    config = ("split q/k RMSNorm + neox RoPE bf16 at prefill size: 16384 tokens, 32 q + "
              "8 kv heads, head_dim 128, eps 1e-6, theta 1e6, cos/sin from int64 "
              "positions U[0,4096) in registers")
    source = "rope.hip"
    kernel = "split_rmsnorm_rope_tok_kernel"
    T, HQ, HKV, HD = 16384, 32, 8, 128
    # qkv in + q/k/v out (bf16) + positions (int64) + q/k weights + inv_freq
    algo_bytes = T * (HQ + 2 * HKV) * HD * 2 * 2 + T * 8 + 2 * HD * 2 + HD // 2 * 4
    CPU_T = 1024

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        hid = (self.HQ + 2 * self.HKV) * self.HD
        self.qkv = _randn((self.T, hid), g, torch.bfloat16)
        self.qw = _randn((self.HD,), g, torch.bfloat16, 0.1, 1.0)
        self.kw = _randn((self.HD,), g, torch.bfloat16, 0.1, 1.0)
        self.pos = torch.randint(0, 4096, (self.T,), generator=g)
        i = torch.arange(0, self.HD, 2, dtype=torch.float64)
        self.inv = (1.0 / (1e6 ** (i / self.HD))).to(torch.float32)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        qw, kw, inv = self.qw.to(dev), self.kw.to(dev), self.inv.to(dev)
        qh, kvh = self.HQ * self.HD, self.HKV * self.HD
        out = []
        for _ in range(n):
            qkv, pos = self.qkv.to(dev), self.pos.to(dev)
            q = torch.empty(self.T, qh, device=dev, dtype=torch.bfloat16)
            k = torch.empty(self.T, kvh, device=dev, dtype=torch.bfloat16)
            v = torch.empty(self.T, kvh, device=dev, dtype=torch.bfloat16)

            def run(qkv=qkv, pos=pos, q=q, k=k, v=v):
                _ok(lib.xk_split_rmsnorm_rope(
                    qkv.data_ptr(), qkv.stride(0), self.T, None, None, self.HD,
                    pos.data_ptr(), _lib.XK_I64, inv.data_ptr(), q.data_ptr(),
                    k.data_ptr(), v.data_ptr(), qw.data_ptr(), None, kw.data_ptr(), None,
                    _lib.XK_BF16, qh, kvh, self.HD, 1e-6, _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import rope as orp
        t = self.CPU_T
        cos, sin = orp.neox_cos_sin(self.pos[:t], self.inv)
        a = (self.qkv[:t], sin, cos, self.qw, self.kw, self.HQ * self.HD,
             self.HKV * self.HD, self.HD, 1e-6)
        return (lambda: orp.split_rmsnorm_rope(*a),
                f"first {t} tokens, fp32 math incl. cos/sin rows", self.T / t)


def varlen_lengths(n, total, lo, hi, gen):
    """n lengths ~ U{lo..hi}, repaired at seeded positions to sum to total."""
    lens = torch.randint(lo, hi + 1, (n,), generator=gen)
    diff = total - int(lens.sum())
    i = 0
    while diff != 0:
        j = i % n
        step = max(-(int(lens[j]) - lo), min(hi - int(lens[j]), diff))
        lens[j] += step
        diff -= step
        i += 1
    return lens


class ConvPrefillCase(Case):
    name = "causal_conv1d_prefill"
    config = ("config 3a: causal_conv1d varlen prefill bf16, 8 sequences "
              "(lengths U[512,3584], 16384 tokens), dim 8192, width 4, SiLU, "
              "w~N(0,0.5), zero initial state")
    source = "conv1d.hip"
    kernel = "conv1d_varlen_kernel"
    T, D, W, NSEQ = 16384, 8192, 4, 8
    # x + y (bf16) + weights + state read/write
    algo_bytes = T * D * 2 * 2 + D * W * 2 + NSEQ * D * (W - 1) * 2 * 2

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        lens = varlen_lengths(self.NSEQ, self.T, 512, 3584, g)
        self.qsl = torch.zeros(self.NSEQ + 1, dtype=torch.int32)
        self.qsl[1:] = torch.cumsum(lens, 0)
        self.mql = int(lens.max())
        self.x = _randn((self.T, self.D), g, torch.bfloat16)
        self.w = _randn((self.D, self.W), g, torch.bfloat16, 0.5)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        w, qsl = self.w.to(dev), self.qsl.to(dev)
        out = []
        for _ in range(n):
            x = self.x.to(dev)
            y = torch.empty_like(x)
            st = torch.zeros(self.NSEQ, self.D, self.W - 1, dtype=torch.bfloat16,
                             device=dev)

            def run(x=x, y=y, st=st):
                _ok(lib.xk_causal_conv1d_varlen(
                    x.data_ptr(), self.D, self.T, y.data_ptr(), self.D,
                    st.data_ptr(), st.stride(0), st.stride(1), st.stride(2),
                    self.NSEQ, self.W - 1, w.data_ptr(), self.W, 1, None,
                    _lib.XK_BF16, qsl.data_ptr(), self.NSEQ, None, 0, 0, None,
                    None, None, self.D, self.W, self.mql, 0, 1, -1,
                    _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import conv1d as oc
        st = torch.zeros(self.NSEQ, self.D, self.W - 1, dtype=torch.bfloat16)
        a = (self.x, st, self.w, None, True, None, self.qsl, self.mql)
        return (lambda: oc.causal_conv1d_update_v2(*a),
                "full config 3a (16384 tokens x 8192), per-sequence F.conv1d fp32", 1.0)


class ConvDecodeCase(Case):
    name = "causal_conv1d_update"
    config = ("config 3b: causal_conv1d decode update bf16, batch 256 x dim 8192, "
              "conv_state [256,8192,3] ~N(0,1), width 4, SiLU, indices arange")
    source = "conv1d.hip"
    kernel = "conv1d_update_w4_kernel"
    timing = "graph"
    B, D, W = 256, 8192, 4
    algo_bytes = B * D * 2 * 2 + B * D * (W - 1) * 2 * 2 + D * W * 2

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.x = _randn((self.B, self.D), g, torch.bfloat16)
        self.state = _randn((self.B, self.D, self.W - 1), g, torch.bfloat16)
        self.w = _randn((self.D, self.W), g, torch.bfloat16, 0.5)
        self.idx = torch.arange(self.B, dtype=torch.int32)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        w, idx = self.w.to(dev), self.idx.to(dev)
        out = []
        for _ in range(n):
            x, st = self.x.to(dev), self.state.to(dev)
            y = torch.empty_like(x)

            def run(x=x, y=y, st=st):
                _ok(lib.xk_causal_conv1d_update(
                    x.data_ptr(), self.D, 1, 1, st.data_ptr(), st.stride(0),
                    st.stride(1), st.stride(2), w.data_ptr(), self.W, 1, None,
                    _lib.XK_BF16, idx.data_ptr(), -1, self.B, y.data_ptr(),
                    self.D, 1, 1, self.B, self.D, 1, self.W, self.W - 1, 1,
                    _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import conv1d as oc
        a = (self.x, self.state, self.w, None, True, self.idx)
        return (lambda: oc.causal_conv1d_update(*a),
                "full config 3b (256 x 8192), fp32", 1.0)


class GdnDecodeInputs:
    """BASELINE config 5 inputs (shared by the fused and unfused cases)."""
    B, H, HV, K, V, W = 256, 16, 32, 128, 128, 4

    def __init__(self):
        import torch.nn.functional as F
        g = torch.Generator().manual_seed(0)
        D = 2 * self.H * self.K + self.HV * self.V
        self.D = D
        self.x = _randn((self.B, D), g, torch.bfloat16)
        self.cs = _randn((self.B, D, self.W - 1), g, torch.bfloat16)
        self.cw = _randn((D, self.W), g, torch.bfloat16, 0.5)
        self.gate = (-F.softplus(torch.randn(self.B, self.HV, generator=g))).to(torch.bfloat16)
        self.beta = torch.sigmoid(torch.randn(self.B, self.HV, generator=g)).to(torch.bfloat16)
        self.state = torch.randn(self.B, self.HV, self.K, self.V, generator=g) * 0.02
        self.idx = torch.arange(self.B, dtype=torch.int32)


class GdnDecodeFusedCase(Case):
    name = "gdn_decode_fused"
    config = ("config 5: recurrent GDN decode fused with causal_conv1d update, "
              "batch 256, 16 qk / 32 v heads, head_dim 128, fp32 state "
              "[256,32,128,128] in place, bf16 mixed_qkv/g/beta")
    source = "gdn_recurrent.hip"
    kernel = "gdn_conv_decode_kernel"
    I = GdnDecodeInputs
    # state r/w + mixed_qkv + conv_state r/w + conv_w + g/beta + o
    algo_bytes = (I.B * I.HV * I.K * I.V * 4 * 2 + I.B * 8192 * 2
                  + I.B * 8192 * 3 * 2 * 2 + 8192 * 4 * 2 + I.B * I.HV * 2 * 2
                  + I.B * I.HV * I.V * 2)

    def __init__(self):
        self.inp = GdnDecodeInputs()

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        a = self.inp
        cw, g, beta, idx = a.cw.to(dev), a.gate.to(dev), a.beta.to(dev), a.idx.to(dev)
        out = []
        for _ in range(n):
            x, cs, st = a.x.to(dev), a.cs.to(dev), a.state.to(dev)
            o = torch.empty(a.B, a.HV, a.V, dtype=torch.bfloat16, device=dev)

            def run(x=x, cs=cs, st=st, o=o):
                _ok(lib.xk_gdn_conv_decode(
                    x.data_ptr(), a.D, cs.data_ptr(), cs.stride(0), cs.stride(1),
                    cs.stride(2), a.B, a.W - 1, cw.data_ptr(), a.W, 1, None,
                    _lib.XK_BF16, a.W, idx.data_ptr(), -1, g.data_ptr(),
                    _lib.XK_BF16, beta.data_ptr(), _lib.XK_BF16, st.data_ptr(),
                    st.stride(0), a.B, idx.data_ptr(), o.data_ptr(), a.B, a.H,
                    a.HV, a.K, a.V, a.K ** -0.5, 1, _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import conv1d as oc
        from oracle import gdn as og
        a = self.inp
        n = a.B  # the whole batch

        def run():
            y, _ = oc.causal_conv1d_update(a.x[:n], a.cs[:n], a.cw, None, True,
                                           a.idx[:n])
            q = y[:, :a.H * a.K].reshape(n, a.H, a.K)
            k = y[:, a.H * a.K:2 * a.H * a.K].reshape(n, a.H, a.K)
            v = y[:, 2 * a.H * a.K:].reshape(n, a.HV, a.V)
            og.recurrent_gdn(q, k, v, a.gate[:n], a.beta[:n], a.K ** -0.5,
                             a.state[:n], T=1, ssm_state_indices=a.idx[:n],
                             dtype=torch.float32)
        return run, ("the full config 5 call: all 256 batch rows (conv update + SiLU, split, "
                     "l2norm, one GDN step; fp32)"), 1.0


class GdnDecodeGatedCase(Case):
    name = "gdn_decode_fused_gating"
    config = ("config 5 from the projection outputs: causal_conv1d update + SiLU + "
              "split + l2norm + GDN gating (g, beta from a, b, A_log, dt_bias) + one "
              "GDN step in one launch, batch 256, 16 qk / 32 v heads, head_dim 128, "
              "fp32 state [256,32,128,128] in place, bf16 mixed_qkv/a/b")
    source = "gdn_recurrent.hip"
    kernel = "gdn_conv_decode_kernel"
    I = GdnDecodeInputs
    # config 5's bytes with a/b (bf16) in place of g/beta, plus A_log / dt_bias
    algo_bytes = GdnDecodeFusedCase.algo_bytes + I.HV * 4 * 2

    def __init__(self):
        self.inp = GdnDecodeInputs()
        g = torch.Generator().manual_seed(1)
        I = GdnDecodeInputs
        self.a = _randn((I.B, I.HV), g, torch.bfloat16)
        self.b = _randn((I.B, I.HV), g, torch.bfloat16)
        self.A_log = torch.randn(I.HV, generator=g)
        self.dt_bias = torch.randn(I.HV, generator=g)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        a = self.inp
        cw, idx = a.cw.to(dev), a.idx.to(dev)
        av, bv = self.a.to(dev), self.b.to(dev)
        al, db = self.A_log.to(dev), self.dt_bias.to(dev)
        out = []
        for _ in range(n):
            x, cs, st = a.x.to(dev), a.cs.to(dev), a.state.to(dev)
            o = torch.empty(a.B, a.HV, a.V, dtype=torch.bfloat16, device=dev)

            def run(x=x, cs=cs, st=st, o=o):
                _ok(lib.xk_gdn_conv_gating_decode(
                    x.data_ptr(), a.D, cs.data_ptr(), cs.stride(0), cs.stride(1),
                    cs.stride(2), a.B, a.W - 1, cw.data_ptr(), a.W, 1, None,
                    _lib.XK_BF16, a.W, idx.data_ptr(), -1, al.data_ptr(), av.data_ptr(),
                    db.data_ptr(), bv.data_ptr(), _lib.XK_BF16, 1.0, 20.0, st.data_ptr(),
                    st.stride(0), a.B, idx.data_ptr(), o.data_ptr(), a.B, a.H,
                    a.HV, a.K, a.V, a.K ** -0.5, 1, _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import conv1d as oc
        from oracle import gating as ogt
        a = self.inp
        n = a.B  # the whole batch

        def run():
            y, _ = oc.causal_conv1d_update(a.x[:n], a.cs[:n], a.cw, None, True,
                                           a.idx[:n])
            q = y[:, :a.H * a.K].reshape(1, n, a.H, a.K)
            k = y[:, a.H * a.K:2 * a.H * a.K].reshape(1, n, a.H, a.K)
            v = y[:, 2 * a.H * a.K:].reshape(1, n, a.HV, a.V)
            ogt.sigmoid_gating_delta_rule_update(
                self.A_log, self.a[:n][None], self.dt_bias, q, k, v, self.b[:n][None],
                a.state[:n], a.idx[:n], torch.arange(n + 1, dtype=torch.int32),
                a.K ** -0.5, True, dtype=torch.float32)
        return (run, "all 256 batch rows (conv update + split + gating + l2norm + GDN step, "
                "fp32)", 1.0)


class GdnRecurrentCase(Case):
    name = "gdn_recurrent"
    config = ("config 5 (unfused a7 form): fused_recurrent_gated_delta_rule, "
              "256 sequences x 1 token, 16 qk / 32 v heads, head_dim 128, "
              "fp32 state in place, in-kernel l2norm")
    source = "gdn_recurrent.hip"
    kernel = "gdn_recurrent_kernel"
    I = GdnDecodeInputs
    # state r/w + q/k/v + g/beta + o
    algo_bytes = (I.B * I.HV * I.K * I.V * 4 * 2 + I.B * (2 * I.H * I.K + I.HV * I.V) * 2
                  + I.B * I.HV * 2 * 2 + I.B * I.HV * I.V * 2)

    def __init__(self):
        a = self.inp = GdnDecodeInputs()
        self.q = a.x[:, :a.H * a.K].reshape(a.B, a.H, a.K).contiguous()
        self.k = a.x[:, a.H * a.K:2 * a.H * a.K].reshape(a.B, a.H, a.K).contiguous()
        self.v = a.x[:, 2 * a.H * a.K:].reshape(a.B, a.HV, a.V).contiguous()

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        a = self.inp
        q, k, v = self.q.to(dev), self.k.to(dev), self.v.to(dev)
        g, beta, idx = a.gate.to(dev), a.beta.to(dev), a.idx.to(dev)
        cu = torch.arange(a.B + 1, dtype=torch.int32, device=dev)
        out = []
        for _ in range(n):
            st = a.state.to(dev)
            o = torch.empty(a.B, a.HV, a.V, dtype=torch.bfloat16, device=dev)

            def run(st=st, o=o):
                _ok(lib.xk_gdn_recurrent(
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.XK_BF16,
                    g.data_ptr(), _lib.XK_BF16, beta.data_ptr(), _lib.XK_BF16,
                    o.data_ptr(), st.data_ptr(), st.stride(0), st.data_ptr(),
                    st.stride(0), a.B, cu.data_ptr(), _lib.XK_I32, idx.data_ptr(),
                    1, 0, None, a.B, 0, a.H, a.HV, a.K, a.V, a.K ** -0.5, 1, 1,
                    _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import gdn as og
        a = self.inp
        n = a.B

        def run():
            og.recurrent_gdn(self.q[:n], self.k[:n], self.v[:n], a.gate[:n],
                             a.beta[:n], a.K ** -0.5, a.state[:n], T=1,
                             ssm_state_indices=a.idx[:n], dtype=torch.float32)
        return run, "all 256 sequences, fp32", 1.0


class GdnGatingCase(Case):
    name = "gdn_gating"
    config = ("next row (npu_fused_gdn_gating) on the prefill shape: 16384 tokens x 32 "
              "v heads, bf16 a/b ~N(0,1), fp32 A_log ~N(0,1) and dt_bias ~N(0,1); "
              "outputs fp32 g and bf16 beta")
    source = "gdn_recurrent.hip"
    kernel = "gdn_gating_kernel"
    timing = "graph"
    R, HV = 16384, 32
    # a, b (bf16) + g (fp32) + beta (bf16) + A_log / dt_bias
    algo_bytes = R * HV * (2 + 2 + 4 + 2) + HV * 8

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.A_log = torch.randn(self.HV, generator=g)
        self.dt_bias = torch.randn(self.HV, generator=g)
        self.a = _randn((self.R, self.HV), g, torch.bfloat16)
        self.b = _randn((self.R, self.HV), g, torch.bfloat16)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        A_log, dt_bias = self.A_log.to(dev), self.dt_bias.to(dev)
        out = []
        for _ in range(n):
            a, b = self.a.to(dev), self.b.to(dev)
            gg = torch.empty(self.R, self.HV, device=dev)
            bo = torch.empty_like(b)

            def run(a=a, b=b, gg=gg, bo=bo):
                _ok(lib.xk_fused_gdn_gating(A_log.data_ptr(), a.data_ptr(), b.data_ptr(),
                                            dt_bias.data_ptr(), gg.data_ptr(), bo.data_ptr(),
                                            self.R, self.HV, 1.0, 20.0, _lib.XK_BF16,
                                            _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import gating as ogt
        a = (self.A_log, self.a, self.b, self.dt_bias)
        return (lambda: ogt.fused_gdn_gating(*a),
                "full shape (16384 x 32), fp32", 1.0)


class GdnSigmoidGatingCase(Case):
    name = "gdn_sigmoid_gating_update"
    config = ("next row (npu_fused_sigmoid_gating_delta_rule_update) on config 5's "
              "decode shapes: 256 sequences x 1 token, 16 qk / 32 v heads, head_dim 128, "
              "fp32 state [256,32,128,128] in place, in-kernel gating from bf16 a/b "
              "and l2norm")
    source = "gdn_recurrent.hip"
    kernel = "gdn_recurrent_kernel"
    I = GdnDecodeInputs
    # state r/w + q/k/v + a/b + o
    algo_bytes = (I.B * I.HV * I.K * I.V * 4 * 2 + I.B * (2 * I.H * I.K + I.HV * I.V) * 2
                  + I.B * I.HV * 2 * 2 + I.B * I.HV * I.V * 2 + I.HV * 8)

    def __init__(self):
        a = self.inp = GdnDecodeInputs()
        g = torch.Generator().manual_seed(1)
        self.q = a.x[:, :a.H * a.K].reshape(a.B, 1, a.H, a.K).contiguous()
        self.k = a.x[:, a.H * a.K:2 * a.H * a.K].reshape(a.B, 1, a.H, a.K).contiguous()
        self.v = a.x[:, 2 * a.H * a.K:].reshape(a.B, 1, a.HV, a.V).contiguous()
        self.ga = _randn((a.B, 1, a.HV), g, torch.bfloat16)
        self.gb = _randn((a.B, 1, a.HV), g, torch.bfloat16)
        self.A_log = torch.randn(a.HV, generator=g)
        self.dt_bias = torch.randn(a.HV, generator=g)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        a = self.inp
        q, k, v = self.q.to(dev), self.k.to(dev), self.v.to(dev)
        ga, gb = self.ga.to(dev), self.gb.to(dev)
        A_log, dt_bias, idx = self.A_log.to(dev), self.dt_bias.to(dev), a.idx.to(dev)
        cu = torch.arange(a.B + 1, dtype=torch.int32, device=dev)
        out = []
        for _ in range(n):
            st = a.state.to(dev)
            o = torch.empty(a.B, 1, a.HV, a.V, dtype=torch.bfloat16, device=dev)

            def run(st=st, o=o):
                _ok(lib.xk_gdn_sigmoid_gating_update(
                    A_log.data_ptr(), ga.data_ptr(), dt_bias.data_ptr(), 1.0, 20.0,
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), gb.data_ptr(), _lib.XK_BF16,
                    o.data_ptr(), st.data_ptr(), st.stride(0), a.B, idx.data_ptr(),
                    cu.data_ptr(), a.B, a.H, a.HV, a.K, a.V, a.K ** -0.5, 1, _lib.XK_BF16,
                    _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import gating as ogt
        a = self.inp
        n = a.B

        def run():
            ogt.sigmoid_gating_delta_rule_update(
                self.A_log, self.ga[:n], self.dt_bias, self.q[:n], self.k[:n], self.v[:n],
                self.gb[:n], a.state[:n], a.idx[:n], torch.arange(n + 1, dtype=torch.int32),
                a.K ** -0.5, True, dtype=torch.float32)
        return run, "all 256 sequences, fp32", 1.0


class QkvzbaSplitCase(Case):
    name = "qkvzba_split"
    config = ("next row (npu_fused_qkvzba_split_reshape_cat) on the prefill shape: "
              "16384 rows, 16 qk / 32 v heads (2 per qk head), head dims 128, bf16 "
              "mixed_qkvz [16384, 12288] and mixed_ba [16384, 64]")
    source = "layout.hip"
    kernel = "qkvzba_split_kernel"
    R, NQK, NV, HD = 16384, 16, 32, 128
    W = NQK * (2 * HD + 2 * (NV // NQK) * HD)
    # every element read once and written once (bf16)
    algo_bytes = R * (W + 2 * NV) * 2 * 2

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.qkvz = _randn((self.R, self.W), g, torch.bfloat16)
        self.ba = _randn((self.R, 2 * self.NV), g, torch.bfloat16)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        out = []
        qkv_dim = 2 * self.NQK * self.HD + self.NV * self.HD
        for _ in range(n):
            qkvz, ba = self.qkvz.to(dev), self.ba.to(dev)
            qkv = torch.empty(self.R, qkv_dim, dtype=torch.bfloat16, device=dev)
            z = torch.empty(self.R, self.NV * self.HD, dtype=torch.bfloat16, device=dev)
            b = torch.empty(self.R, self.NV, dtype=torch.bfloat16, device=dev)
            a = torch.empty_like(b)

            def run(qkvz=qkvz, ba=ba, qkv=qkv, z=z, b=b, a=a):
                _ok(lib.xk_fused_qkvzba_split_reshape_cat(
                    qkvz.data_ptr(), self.W, ba.data_ptr(), 2 * self.NV, qkv.data_ptr(),
                    z.data_ptr(), b.data_ptr(), a.data_ptr(), self.R, self.NQK, self.NV,
                    self.HD, self.HD, _lib.XK_BF16, _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import layout as ol
        a = (self.qkvz, self.ba, self.NQK, self.NV, self.HD, self.HD)
        return (lambda: ol.fused_qkvzba_split_reshape_cat(*a), "full shape, copies", 1.0)


def chunk_gdn_flops(tokens, HV, K=128, V=128, C=64):
    """Algorithmic FLOPs of the chunked gated delta rule per call, summed
    per 64-token chunk and v-head: K K^T, Q K^T (2C^2K each), W = A(k b e^g)
    (2C^2K), U = A(v b) and (QK^T) Vn (2C^2V each), W S, Q S and the state
    update K^T Vn (2CKV each), and the triangular inverse (C^3/3)."""
    per_chunk = 3 * 2 * C * C * K + 2 * 2 * C * C * V + 3 * 2 * C * K * V + C ** 3 // 3
    return tokens * HV * per_chunk // C


class GdnChunkCase(Case):
    name = "gdn_chunk_prefill"
    config = ("config 4: chunked gated delta rule prefill bf16, 8 sequences "
              "(lengths U[512,3584], 16384 tokens), 16 qk / 32 v heads, head_dim "
              "128, chunk 64, q/k l2-normalised, g=-softplus(N(0,1)) fp32, "
              "beta=sigmoid(N(0,1)) bf16, h0~N(0,0.02) fp32, outputs o + final state")
    source = "gdn_chunk.hip"
    kernel = "gdn_chunk_state8_kernel"
    T, NSEQ, H, HV, K, V = 16384, 8, 16, 32, 128, 128
    # q/k + v + o (bf16) + g (fp32) + beta (bf16) + h0/ht (fp32)
    algo_bytes = (T * H * K * 2 * 2 + T * HV * V * 2 * 2 + T * HV * (4 + 2)
                  + NSEQ * HV * K * V * 4 * 2)
    algo_flops = chunk_gdn_flops(T, HV, K, V)
    tokens = T

    def __init__(self):
        import torch.nn.functional as F
        g = torch.Generator().manual_seed(0)
        lens = varlen_lengths(self.NSEQ, self.T, 512, 3584, g)
        self.cu = torch.zeros(self.NSEQ + 1, dtype=torch.int32)
        self.cu[1:] = torch.cumsum(lens, 0)

        def unit(x):
            return (x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
        self.q = unit(torch.randn(self.T, self.H, self.K, generator=g))
        self.k = unit(torch.randn(self.T, self.H, self.K, generator=g))
        self.v = _randn((self.T, self.HV, self.V), g, torch.bfloat16)
        self.g = -F.softplus(torch.randn(self.T, self.HV, generator=g))
        self.beta = torch.sigmoid(torch.randn(self.T, self.HV, generator=g)).to(torch.bfloat16)
        self.h0 = torch.randn(self.NSEQ, self.HV, self.K, self.V, generator=g) * 0.02

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        cu = self.cu.to(dev)
        wsb = lib.xk_gdn_chunk_workspace_bytes(self.T, self.NSEQ, self.HV)
        out = []
        for _ in range(n):
            q, k, v = self.q.to(dev), self.k.to(dev), self.v.to(dev)
            g, beta, h0 = self.g.to(dev), self.beta.to(dev), self.h0.to(dev)
            o = torch.empty_like(v)
            ht = torch.empty_like(h0)
            ws = torch.empty(wsb, dtype=torch.uint8, device=dev)

            def run(q=q, k=k, v=v, g=g, beta=beta, h0=h0, o=o, ht=ht, ws=ws):
                _ok(lib.xk_gdn_chunk_fwd(
                    q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.XK_BF16,
                    g.data_ptr(), _lib.XK_F32, beta.data_ptr(), _lib.XK_BF16,
                    o.data_ptr(), h0.data_ptr(), ht.data_ptr(), cu.data_ptr(),
                    _lib.XK_I32, self.NSEQ, self.T, self.H, self.HV, self.K,
                    self.V, self.K ** -0.5, 0, ws.data_ptr(), wsb, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import gdn as og
        # The whole workload (about 2 s per call on 16 host threads), not a
        # scaled sample of it.
        a = (self.q[None], self.k[None], self.v[None], self.g[None], self.beta[None],
             self.K ** -0.5, self.h0, self.cu)
        return (lambda: og.chunk_gdn(*a),
                f"the full config 4 call: all 16384 tokens and {self.HV} v-heads, fp32 "
                "chunked form of the reference golden", 1.0)


class GdnChunkStagedCase(GdnChunkCase):
    """Config 4 through the six stage entry points in the reference's order
    (npu_triton_chunk_gated_delta_rule.cpp:556-642): cumsum, scaled K K^T,
    solve_tril (bf16 Ai), w/u, the state recurrence (bf16 h snapshots and
    v_new) and the output, with every intermediate in HBM."""
    name = "gdn_chunk_staged"
    config = ("config 4 through the stage-by-stage API (chunk_local_cumsum, "
              "scaled_dot_kkt, solve_tril, recompute_w_u, fwd_h, fwd_o), the "
              "reference's intermediates (A, Ai, w, u, h, v_new) kept in HBM")
    source = "gdn_stages.hip"
    kernel = "chunk_fwd_h8_kernel"

    def nchunks(self):
        lens = (self.cu[1:] - self.cu[:-1]).tolist()
        return sum(-(-int(x) // 64) for x in lens)

    def stage_io(self):
        """(entry point, kernel, bytes of the stage's own inputs and outputs
        at their dtypes) per stage, in pipeline order: the stage API keeps
        its intermediates in HBM by definition, so each stage's roofline is
        its own traffic."""
        T, H, HV, K, V, N = self.T, self.H, self.HV, self.K, self.V, self.NSEQ
        nt = self.nchunks()
        cu = (N + 1) * 4
        k_b = T * H * K * 2          # k (bf16), also q
        v_b = T * HV * V * 2         # v, u, v_new, o (bf16)
        w_b = T * HV * K * 2         # w (bf16)
        g_b = T * HV * 4             # g, g_cumsum (fp32)
        bt_b = T * HV * 2            # beta (bf16)
        A_b = T * HV * 64 * 4        # A (fp32)
        Ai_b = T * HV * 64 * 2       # Ai (bf16)
        h_b = nt * HV * K * V * 2    # h snapshots (bf16)
        s_b = N * HV * K * V * 4     # h0 / ht (fp32)
        return [
            ("chunk_local_cumsum", "chunk_cumsum_scan_kernel", 2 * g_b + cu),
            ("chunk_scaled_dot_kkt", "chunk_kkt_kernel", k_b + bt_b + g_b + A_b + cu),
            ("solve_tril", "solve_tril_kernel", A_b + Ai_b + cu),
            ("recompute_w_u", "recompute_w_u_kernel",
             k_b + v_b + bt_b + g_b + Ai_b + w_b + v_b + cu),
            ("chunk_fwd_h", "chunk_fwd_h8_kernel", k_b + w_b + v_b + g_b + 2 * s_b + h_b + v_b + cu),
            ("chunk_fwd_o", "chunk_fwd_o_kernel", 2 * k_b + v_b + h_b + g_b + v_b + cu),
        ]

    def stage_sets(self, dev, n):
        """n buffer sets, each a list of the six stage closures (in order)."""
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        cu = self.cu.to(dev)
        nt = self.nchunks()
        wsb = lib.xk_gdn_stage_workspace_bytes(self.NSEQ)
        T, H, HV, K, V = self.T, self.H, self.HV, self.K, self.V
        bf, f32 = torch.bfloat16, torch.float32
        I32, BF, F32 = _lib.XK_I32, _lib.XK_BF16, _lib.XK_F32
        out = []
        for _ in range(n):
            q, k, v = self.q.to(dev), self.k.to(dev), self.v.to(dev)
            g, beta, h0 = self.g.to(dev), self.beta.to(dev), self.h0.to(dev)
            b = dict(
                gc=torch.empty(T, HV, dtype=f32, device=dev),
                A=torch.empty(T, HV, 64, dtype=f32, device=dev),
                Ai=torch.empty(T, HV, 64, dtype=bf, device=dev),
                w=torch.empty(T, HV, K, dtype=bf, device=dev),
                u=torch.empty(T, HV, V, dtype=bf, device=dev),
                h=torch.empty(nt, HV, K, V, dtype=bf, device=dev),
                vn=torch.empty(T, HV, V, dtype=bf, device=dev),
                ht=torch.empty_like(h0), o=torch.empty_like(v),
                ws=torch.empty(wsb, dtype=torch.uint8, device=dev))
            ws = b["ws"].data_ptr()

            def cumsum(g=g, b=b, ws=ws):
                _ok(lib.xk_chunk_local_cumsum(g.data_ptr(), F32, b["gc"].data_ptr(), T, HV,
                                              cu.data_ptr(), I32, self.NSEQ, 64, _cur_stream()),
                    lib)

            def kkt(k=k, beta=beta, b=b, ws=ws):
                _ok(lib.xk_chunk_scaled_dot_kkt(k.data_ptr(), BF, beta.data_ptr(), BF,
                                                b["gc"].data_ptr(), b["A"].data_ptr(), T, H, HV,
                                                K, cu.data_ptr(), I32, self.NSEQ, ws, wsb,
                                                _cur_stream()), lib)

            def tril(b=b, ws=ws):
                _ok(lib.xk_solve_tril(b["A"].data_ptr(), b["Ai"].data_ptr(), BF, T, HV,
                                      cu.data_ptr(), I32, self.NSEQ, ws, wsb, _cur_stream()), lib)

            def wu(k=k, v=v, beta=beta, b=b, ws=ws):
                _ok(lib.xk_recompute_w_u(k.data_ptr(), v.data_ptr(), BF, beta.data_ptr(), BF,
                                         b["gc"].data_ptr(), b["Ai"].data_ptr(), BF,
                                         b["w"].data_ptr(), b["u"].data_ptr(), T, H, HV, K, V,
                                         cu.data_ptr(), I32, self.NSEQ, ws, wsb, _cur_stream()),
                    lib)

            def fwd_h(k=k, h0=h0, b=b, ws=ws):
                _ok(lib.xk_chunk_fwd_h(k.data_ptr(), b["w"].data_ptr(), b["u"].data_ptr(), BF,
                                       b["gc"].data_ptr(), h0.data_ptr(), b["h"].data_ptr(), nt,
                                       b["vn"].data_ptr(), b["ht"].data_ptr(), T, H, HV, K, V,
                                       cu.data_ptr(), I32, self.NSEQ, ws, wsb, _cur_stream()),
                    lib)

            def fwd_o(q=q, k=k, b=b, ws=ws):
                _ok(lib.xk_chunk_fwd_o(q.data_ptr(), k.data_ptr(), b["vn"].data_ptr(),
                                       b["h"].data_ptr(), nt, BF, b["gc"].data_ptr(),
                                       b["o"].data_ptr(), self.K ** -0.5, T, H, HV, K, V,
                                       cu.data_ptr(), I32, self.NSEQ, ws, wsb, _cur_stream()),
                    lib)
            out.append([cumsum, kkt, tril, wu, fwd_h, fwd_o])
        return out

    def sets(self, dev, n):
        out = []
        for st in self.stage_sets(dev, n):
            def run(st=st):
                for f in st:
                    f()
            out.append(run)
        return out

    def cpu(self):
        return None  # the same workload as gdn_chunk_prefill: its CPU line is reused


class L2NormCase(Case):
    name = "l2norm_last_dim"
    config = ("a6a (npu_l2norm_last_dim) on the prefill shape: q or k of config 4 as "
              "rows, bf16 [262144, 128] (16384 tokens x 16 heads), eps 1e-6, bf16 out")
    source = "norm.hip"
    kernel = "l2norm_team_kernel"
    timing = "graph"
    R, C = 16384 * 16, 128
    algo_bytes = R * C * 2 * 2

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.x = _randn((self.R, self.C), g, torch.bfloat16)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        lib = _lib.lib()
        out = []
        for _ in range(n):
            x = self.x.to(dev)
            y = torch.empty_like(x)

            def run(x=x, y=y):
                _ok(lib.xk_l2norm_last_dim(x.data_ptr(), y.data_ptr(), self.R, self.C, 1e-6,
                                           _lib.XK_BF16, _lib.XK_BF16, _cur_stream()), lib)
            out.append(run)
        return out

    def cpu(self):
        from oracle import norm as on
        x = self.x
        return (lambda: on.l2norm_last_dim(x, 1e-6), "full shape, fp32 math on bf16 input", 1.0)


_MEASURE = None


def measure_lib():
    """libxk_measure.so (bench.py's reference kernels), built next to
    libxk.so by torch_npu_ops_amd/_build.py."""
    global _MEASURE
    if _MEASURE is None:
        import ctypes
        path = os.path.join(REPO, "torch_npu_ops_amd", "libxk_measure.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
        lib = ctypes.CDLL(path)
        lib.xkm_empty.argtypes = [ctypes.c_void_p]
        lib.xkm_empty.restype = ctypes.c_int
        lib.xkm_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                 ctypes.c_void_p]
        lib.xkm_copy.restype = ctypes.c_int
        lib.xkm_tail_rw.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                    ctypes.c_int64, ctypes.c_void_p]
        lib.xkm_tail_rw.restype = ctypes.c_int
        lib.xkm_tile_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        lib.xkm_tile_copy.restype = ctypes.c_int
        _MEASURE = lib
    return _MEASURE


class CopyFloorCase(Case):
    """A plain device copy moving `moved` bytes (half read, half written):
    the floor of an HBM-bound kernel with the same traffic, timed in the
    same harness (graph replay, buffers rotated past the Infinity Cache)."""
    timing = "graph"
    kernel = "copy16_kernel"

    def __init__(self, moved):
        self.nbytes = max(16, (moved // 2) // 16 * 16)
        self.algo_bytes = 2 * self.nbytes
        self.name = f"copy_{self.algo_bytes}"
        self.config = f"plain device copy of {self.nbytes} B ({self.algo_bytes} B moved)"

    def sets(self, dev, n):
        lib = measure_lib()
        out = []
        for _ in range(n):
            src = torch.empty(self.nbytes, dtype=torch.uint8, device=dev).fill_(1)
            dst = torch.empty_like(src)

            def run(src=src, dst=dst):
                _ok(lib.xkm_copy(src.data_ptr(), dst.data_ptr(), self.nbytes, _cur_stream()),
                    lib)
            out.append(run)
        return out


class TailFloorCase(Case):
    """In-place read-modify-write of the last `tail` bytes of `rows` rows of
    `pitch` bytes, one 16-byte vector per lane and nothing else: the floor
    of an op whose HBM traffic has that strided pattern (rope_inplace),
    timed in the same harness."""
    timing = "graph"
    kernel = "tail_rw_kernel"

    def __init__(self, rows, pitch, tail):
        self.rows, self.pitch, self.tail = rows, pitch, tail
        self.algo_bytes = 2 * rows * tail
        self.name = f"tail_rw_{rows}x{tail}of{pitch}"
        self.config = f"in-place rewrite of the last {tail} B of {rows} rows of {pitch} B"

    def sets(self, dev, n):
        lib = measure_lib()
        out = []
        for _ in range(n):
            x = torch.zeros(self.rows * self.pitch, dtype=torch.uint8, device=dev)

            def run(x=x):
                _ok(lib.xkm_tail_rw(x.data_ptr(), self.rows, self.pitch, self.tail,
                                    _cur_stream()), lib)
            out.append(run)
        return out


class TileFloorCase(Case):
    """A [rows, slices x width] array copied by tiles of 64 rows x one
    width-byte slice, one block per tile, slices of a row group adjacent in
    the grid: the access pattern of the chunked-GDN stage kernels (a
    (chunk, head) piece of a [T, H, 128] bf16 tensor), as a plain copy."""
    timing = "graph"
    kernel = "tile_copy_kernel"

    def __init__(self, rows, slices, width):
        self.rows, self.slices, self.width = rows, slices, width
        self.nbytes = rows * slices * width
        self.algo_bytes = 2 * self.nbytes
        self.name = f"tile_copy_{rows}x{slices}x{width}"
        self.config = (f"copy of a [{rows}, {slices} x {width} B] array by 64-row x {width} B "
                       f"tiles ({self.algo_bytes} B moved)")

    def sets(self, dev, n):
        lib = measure_lib()
        out = []
        for _ in range(n):
            src = torch.empty(self.nbytes, dtype=torch.uint8, device=dev).fill_(1)
            dst = torch.empty_like(src)

            def run(src=src, dst=dst):
                _ok(lib.xkm_tile_copy(src.data_ptr(), dst.data_ptr(), self.rows, self.slices,
                                      self.width, _cur_stream()), lib)
            out.append(run)
        return out


class EmptyKernelCase(Case):
    """The launch floor: an empty kernel, timed like the small ops."""
    name = "empty_kernel"
    timing = "graph"
    kernel = "empty_kernel"
    algo_bytes = 0

    def sets(self, dev, n):
        lib = measure_lib()
        return [lambda: _ok(lib.xkm_empty(_cur_stream()), lib)] * n


CASES = {c.name: c for c in (LayerNormCase, GemmaCase, RopeCase, RopePrefillCase,
                             ConvPrefillCase,
                             ConvDecodeCase, GdnDecodeFusedCase, GdnDecodeGatedCase,
                             GdnRecurrentCase,
                             GdnChunkCase, GdnChunkStagedCase, GdnGatingCase,
                             GdnSigmoidGatingCase, GatedRmsNormCase, QkvzbaSplitCase,
                             RopeInplaceCase, L2NormCase)}
HEADLINE = "layer_norm_fwd"


# ---------------------------------------------------------------------------
# Timing
# ---------------------------------------------------------------------------
# Untimed wall time each op runs before its warm-up calls.  The GPU raises
# its clocks only after some tens of milliseconds of sustained load: on
# MI355X a 47 us layer_norm_fwd call measures ~51 us until about 20 ms of
# back-to-back calls have run, and ~46.7 us from then on.  The settle phase
# makes every op's number the steady-state rate a serving loop sees.
SETTLE_S = 0.1


def _settle(fn):
    """Call fn() back to back until SETTLE_S of wall time has passed (the
    GPU stays busy: calls are queued in batches and synchronised only
    between batches)."""
    end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def time_gpu(case: Case, dev, steps: int, warmup: int, eager: bool):
    """Mean per-call time (ms) of `steps` back-to-back calls, median of
    three timed repetitions, after a clock-settle phase and `warmup`
    untimed calls."""
    per_set = max(case.algo_bytes, 1)
    nsets = max(2, min(MAX_SETS, -(-ROTATE_BYTES // per_set)))
    if case.algo_bytes == 0:
        nsets = 2
    runs = case.sets(dev, nsets)
    ms = time_runs(runs, dev, steps, warmup, eager)
    del runs
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return ms


def time_runs(runs, dev, steps: int, warmup: int, eager: bool):
    """time_gpu's timing of closures that rotate over len(runs) buffer sets."""
    nsets = len(runs)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(warmup):
            runs[i % nsets]()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    if eager:
        ctr = [0]

        def one():
            runs[ctr[0] % nsets]()
            ctr[0] += 1
        _settle(one)
        reps = []
        for _ in range(3):
            t0.record()
            for i in range(steps):
                runs[i % nsets]()
            t1.record()
            torch.cuda.synchronize()
            reps.append(t0.elapsed_time(t1) / steps)
        ms = statistics.median(reps)
    else:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(steps):
                runs[i % nsets]()
        graph.replay()
        torch.cuda.synchronize()
        _settle(graph.replay)
        reps = []
        for _ in range(3):
            t0.record()
            graph.replay()
            t1.record()
            torch.cuda.synchronize()
            reps.append(t0.elapsed_time(t1) / steps)
        ms = statistics.median(reps)
        del graph
    return ms


def time_stages(case, dev, steps: int, warmup: int):
    """Per-stage time (ms) of a staged case: every buffer set runs the whole
    pipeline once (so each stage's inputs hold real intermediates), then
    each stage is timed alone, eagerly, over the sets."""
    nsets = max(2, min(MAX_SETS, -(-ROTATE_BYTES // max(case.algo_bytes, 1))))
    sets = case.stage_sets(dev, nsets)
    for st in sets:
        for f in st:
            f()
    torch.cuda.synchronize()
    out = []
    for i in range(len(sets[0])):
        out.append(time_runs([st[i] for st in sets], dev, steps, warmup, True))
    del sets
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def time_cpu(case: Case):
    """(seconds per full call, sample description, runs, scale) of the op's
    CPU baseline: one warm-up, then the median of at least three timed runs
    (up to five within 20 s), times `scale` when the closure runs a stated
    sample of the call (scale 1: the whole call is timed).  None when the
    case has no CPU closure of its own."""
    torch.set_num_threads(cpu_threads())
    got = case.cpu()
    if got is None:
        return None
    run, sample, scale = got
    run()  # warm-up
    ts = []
    budget_end = time.perf_counter() + 20.0
    while len(ts) < 3 or (time.perf_counter() < budget_end and len(ts) < 5):
        t = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t)
        if time.perf_counter() > budget_end:
            break
    return statistics.median(ts) * scale, sample, len(ts), scale


def cpu_line(case: Case, gpu_us: float):
    """The op line's cpu_baseline object (None if the case has no CPU
    closure)."""
    got = time_cpu(case)
    if got is None:
        return None
    sec, sample, nrun, scale = got
    per_tok = getattr(case, "tokens", 0)
    line = {"value": round(per_tok / sec) if per_tok else round(case.algo_bytes / sec / 1e9, 3),
            "unit": "tokens/s" if per_tok else "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": sample, "scale": scale, "runs": nrun,
            "ms_per_call": round(sec * 1e3, 3),
            "gpu_speedup": round(sec * 1e6 / gpu_us, 1),
            **cpu_host()}
    print(f"[bench] cpu baseline {case.name}: {sec*1e3:.1f} ms/call"
          + (f" (sample x {scale:g})" if scale != 1.0 else " (whole call)"),
          file=sys.stderr, flush=True)
    return line


def source_sha(fname):
    """Hash of a kernel source file and the headers every kernel includes:
    recorded with each traffic measurement, so a measurement taken before a
    kernel changed is not reported as the current kernel's."""
    import hashlib
    import glob
    csrc = os.path.join(REPO, "torch_npu_ops_amd", "csrc")
    h = hashlib.sha256()
    for path in [os.path.join(csrc, fname)] + sorted(glob.glob(os.path.join(csrc, "*.h"))):
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


TRAFFIC_JSON = os.path.join(REPO, "profiles", "hbm_traffic_all_configs.json")


def measured_traffic(case):
    """HBM bytes per dispatch of case.kernel from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE runs (scaled by a plain copy) recorded in TRAFFIC_JSON, or
    None, with a warning, when there is no entry or it was measured on other
    kernel sources than the current ones."""
    if not os.path.exists(TRAFFIC_JSON):
        print(f"[bench] warning: {TRAFFIC_JSON} missing; roofline.traffic is null",
              file=sys.stderr)
        return None
    with open(TRAFFIC_JSON) as f:
        t = json.load(f)
    val = t.get("traffic_bytes", {}).get(case.kernel)
    if val is None:
        print(f"[bench] warning: no traffic entry for {case.kernel}; roofline.traffic is null",
              file=sys.stderr)
        return None
    rec = t.get("sources", {}).get(case.source)
    if rec != source_sha(case.source):
        print(f"[bench] warning: the traffic of {case.kernel} was measured on another "
              f"version of {case.source}; roofline.traffic is null", file=sys.stderr)
        return None
    return round(val)


def cpu_host():
    """What the CPU baseline ran on."""
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = None
    return {"os_cpu_count": os.cpu_count(), "affinity_cpus": aff,
            "cgroup_cpus": _cgroup_cpus(), "torch_threads": torch.get_num_threads(),
            "cpu_model": _cpu_model()}


COPY_BYTES = 256 << 20


def copy_calibration(dev, steps):
    """Plain device copies of COPY_BYTES (read COPY_BYTES, write COPY_BYTES)
    between buffers that rotate over 1 GiB, so that rocprofv3's FETCH_SIZE
    and WRITE_SIZE per dispatch can be scaled to bytes."""
    n = COPY_BYTES // 4
    bufs = [torch.empty(n, dtype=torch.float32, device=dev).uniform_() for _ in range(5)]
    torch.cuda.synchronize()
    for i in range(steps):
        bufs[(i + 1) % 5].copy_(bufs[i % 5])
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_BYTES, "dispatches": steps}))


def floors(dev, steps, warmup, moved_list):
    """Launch floor (empty kernel) and same-traffic copy floors, in the
    graph harness of the small ops."""
    out = {"empty_kernel_us": round(time_gpu(EmptyKernelCase(), dev, steps, warmup, False)
                                    * 1e3, 2)}
    copies = {}
    for moved in moved_list:
        c = CopyFloorCase(moved)
        us = time_gpu(c, dev, steps, warmup, False) * 1e3
        copies[str(c.algo_bytes)] = {"us": round(us, 2),
                                     "GB/s": round(c.algo_bytes / (us * 1e-6) / 1e9, 1)}
        print(f"[bench] floor: copy moving {c.algo_bytes} B: {us:.2f} us", file=sys.stderr,
              flush=True)
    out["copies"] = copies
    return out


# ---------------------------------------------------------------------------
# Profile summaries (profiles/): rocprofv3 output of the runs listed in
# PROFILE_COMMANDS, summarised into the kernel-duration and HBM-traffic tables
# and the traffic JSON that measured_traffic() reads.
# ---------------------------------------------------------------------------
PROFILE_COMMANDS = [
    ("trace", "rocprofv3 --kernel-trace --stats -f csv -d <out>/trace -o run -- "
              "python3 <repo>/bench.py > <out>/trace_bench.json"),
    ("FETCH_SIZE", "rocprofv3 --pmc FETCH_SIZE -f csv -d <out>/FETCH_SIZE -o p -- "
                   "python3 <repo>/bench.py --no-cpu --eager --steps 3 --warmup 1"),
    ("WRITE_SIZE", "rocprofv3 --pmc WRITE_SIZE -f csv -d <out>/WRITE_SIZE -o p -- "
                   "python3 <repo>/bench.py --no-cpu --eager --steps 3 --warmup 1"),
    ("copy_FETCH_SIZE", "rocprofv3 --pmc FETCH_SIZE -f csv -d <out>/copy_FETCH_SIZE -o p -- "
                        "python3 <repo>/bench.py --copy-calibration --steps 5"),
    ("copy_WRITE_SIZE", "rocprofv3 --pmc WRITE_SIZE -f csv -d <out>/copy_WRITE_SIZE -o p -- "
                        "python3 <repo>/bench.py --copy-calibration --steps 5"),
]

# Kernels of each multi-kernel op, in launch order (per-call time against the
# sum of their per-dispatch medians).
OP_KERNELS = {
    # Up to 64 sequences (config 4 has 8) no offsets kernel runs.
    "gdn_chunk_prefill": ["gdn_chunk_prep_kernel", "gdn_chunk_state8_kernel"],
}


def kernel_label(raw):
    """Short kernel name of a rocprofv3 kernel name (mangled or not): the
    kernel identifier, with ln_tile_kernel's template arguments and
    chunk_offsets_kernel's parameter type kept."""
    import re
    m = re.search(r"chunk_offsets_kernel<xk::\(anonymous namespace\)::(\w+)>", raw)
    if m:
        return f"chunk_offsets_kernel<{m.group(1)}>"
    m = re.search(r"ln_tile_kernelI\w+?Li\d+ELi(\d+)ELi(\d+)ELb(\d)ELb(\d)E", raw)
    if m:
        return f"ln_tile_kernel<TPG={m.group(1)},NV={m.group(2)},z={m.group(3)}>"
    m = re.search(r"\d+([a-z][a-z0-9_]*_kernel)I", raw)  # mangled template kernel
    if m:
        return m.group(1)
    m = re.search(r"([a-z][a-z0-9_]*_kernel)\b", raw)
    if m:
        return m.group(1)
    for pat in (r"(__amd_rocclr_copyBuffer)", r"(FillFunctor)", r"(arange)"):
        m = re.search(pat, raw)
        if m:
            return m.group(1)
    return raw[:50]


def _trace_durations(out_dir):
    """Per-dispatch kernel durations (us) by kernel label, from the
    --kernel-trace CSV of the trace run."""
    import csv
    import collections
    dur = collections.defaultdict(list)
    path = glob_one(os.path.join(out_dir, "trace", "**", "run_kernel_trace.csv"))
    for r in csv.DictReader(open(path)):
        dur[kernel_label(r["Kernel_Name"])].append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return dur


def glob_one(pattern):
    import glob
    hits = sorted(glob.glob(pattern, recursive=True))
    if not hits:
        raise FileNotFoundError(pattern)
    return hits[0]


def summarize_profile(out_dir):
    """Writes profiles/kernel_durations_all_configs.md,
    profiles/hbm_traffic_all_configs.md and TRAFFIC_JSON from the rocprofv3
    output directories of PROFILE_COMMANDS under out_dir."""
    import csv
    import collections
    import glob
    dur = _trace_durations(out_dir)
    stats = []
    for k, v in dur.items():
        stats.append((k, len(v), statistics.median(v), statistics.mean(v), min(v), max(v)))
    stats.sort(key=lambda x: -x[2])
    bench_line = None
    bpath = os.path.join(out_dir, "trace_bench.json")
    if os.path.exists(bpath):
        for ln in open(bpath):
            if ln.startswith("{"):
                bench_line = json.loads(ln)

    def pmc(sub, counter):
        acc = collections.defaultdict(list)
        for r in csv.DictReader(open(glob_one(os.path.join(out_dir, sub, "**",
                                                           "p_counter_collection.csv")))):
            if r["Counter_Name"] == counter:
                acc[kernel_label(r["Kernel_Name"])].append(float(r["Counter_Value"]))
        return {k: statistics.mean(v) for k, v in acc.items()}

    fetch, write = pmc("FETCH_SIZE", "FETCH_SIZE"), pmc("WRITE_SIZE", "WRITE_SIZE")
    cf, cw = pmc("copy_FETCH_SIZE", "FETCH_SIZE"), pmc("copy_WRITE_SIZE", "WRITE_SIZE")
    copyk = max(cf, key=cf.get)
    ff = COPY_BYTES / (cf[copyk] * 1024)
    wf = COPY_BYTES / (cw[copyk] * 1024)
    algo = {}  # kernel -> algorithmic bytes of the ops it runs alone
    kernel_ops = collections.defaultdict(list)
    for c in CASES.values():
        kernel_ops[c.kernel].append(c.name)
        algo.setdefault(c.kernel, []).append(c.algo_bytes)
    for op, ks in OP_KERNELS.items():
        for k in ks:
            if op not in kernel_ops[k]:
                kernel_ops[k].append(op)
    traffic = {k: fetch[k] * 1024 * ff + write[k] * 1024 * wf
               for k in fetch if k in write}
    csrc = os.path.join(REPO, "torch_npu_ops_amd", "csrc")
    sources = {os.path.basename(f): source_sha(os.path.basename(f))
               for f in sorted(glob.glob(os.path.join(csrc, "*.hip")))}
    with open(TRAFFIC_JSON, "w") as f:
        json.dump({"fetch_factor": ff, "write_factor": wf, "sources": sources,
                   "traffic_bytes": traffic}, f, indent=1)
    prof = os.path.join(REPO, "profiles")
    cmds = dict(PROFILE_COMMANDS)
    ops = bench_line["ops"] if bench_line else {}
    with open(os.path.join(prof, "kernel_durations_all_configs.md"), "w") as f:
        f.write("# Kernel durations, all BASELINE configs\n\nCommand (repo root on the GPU box; "
                "`cd /tmp && export TMPDIR=/tmp` first):\n\n    " + cmds["trace"] + "\n\n"
                "bench.py's default run (clock-settle phase, warm-up, 3 x 50 timed calls per op "
                "on buffer sets rotated past the Infinity Cache; small ops graph-replayed, plus "
                "their same-traffic copies; the stage-by-stage line also times each stage alone).  "
                "Per-dispatch durations come from the kernel-trace CSV; the median is the "
                "steady-state figure (the first tens of dispatches of an op run before the "
                "clocks settle).  The last column is the per-call time that the same run's bench "
                "line reports (HIP events around back-to-back calls), so both come from one "
                "process on one box.  Summarised by `python3 bench.py --summarize-profile "
                "<out>`.\n\n"
                "| kernel | dispatches | median us | mean us | min us | max us | bench ops | "
                "bench us per call (same run) |\n|---|---|---|---|---|---|---|---|\n")
        for k, c, med, mean, mn, mx in stats:
            names = kernel_ops.get(k, [])
            per_call = ", ".join(f"{ops[n]['us_per_call']:.2f}" for n in names if n in ops)
            f.write(f"| {k} | {c} | {med:.2f} | {mean:.2f} | {mn:.2f} | {mx:.2f} | "
                    f"{', '.join(names) or '-'} | {per_call or '-'} |\n")
        for op, ks in OP_KERNELS.items():
            if all(k in dur for k in ks) and op in ops:
                meds = [statistics.median(dur[k]) for k in ks]
                f.write(f"\n{op}: the per-dispatch medians of its kernels ("
                        + " + ".join(f"{k} {m:.2f}" for k, m in zip(ks, meds))
                        + f") sum to {sum(meds):.2f} us; the same run's bench line measures "
                        f"{ops[op]['us_per_call']:.2f} us per call.\n")
        if bench_line:
            f.write("\nThe same run's bench line (per op: us per call and fraction of the HBM "
                    "peak):\n\n| op | us per call | GB/s | frac |\n|---|---|---|---|\n")
            for n, o in ops.items():
                f.write(f"| {n} | {o['us_per_call']:.2f} | {o['GB/s']:.1f} | "
                        f"{o['roofline']['frac']:.4f} |\n")
    with open(os.path.join(prof, "hbm_traffic_all_configs.md"), "w") as f:
        f.write("# HBM traffic per dispatch vs algorithmic bytes, all BASELINE configs\n\n"
                "Commands (repo root on the GPU box; `cd /tmp && export TMPDIR=/tmp` first; "
                "each counter in its own run):\n\n")
        for key in ("FETCH_SIZE", "WRITE_SIZE", "copy_FETCH_SIZE", "copy_WRITE_SIZE"):
            f.write("    " + cmds[key] + "\n")
        f.write(f"\nCalibration: a plain {COPY_BYTES >> 20} MiB device copy (`{copyk}`) reads "
                f"FETCH_SIZE = {cf[copyk]:.0f} KiB and WRITE_SIZE = {cw[copyk]:.0f} KiB per "
                f"dispatch, so bytes = FETCH_SIZE x 1024 x {ff:.3f} + WRITE_SIZE x 1024 x "
                f"{wf:.3f}.  Summarised by `python3 bench.py --summarize-profile <out>`, which "
                "also writes hbm_traffic_all_configs.json with a hash of every kernel source; "
                "bench.py reports a kernel's traffic only while its source is unchanged.  For "
                "an op made of several kernels (gdn_chunk_prefill, gdn_chunk_staged) the ratio "
                "compares one kernel's traffic with the whole op's algorithmic bytes.\n\n"
                "| kernel | FETCH KiB | WRITE KiB | HBM MB | algorithmic MB (bench op) | "
                "traffic / algorithmic |\n|---|---|---|---|---|---|\n")
        for k, *_ in stats:
            if k not in traffic:
                continue
            a = algo.get(k)
            ratio = f"{traffic[k] / statistics.mean(a):.3f}" if a else "-"
            alg = f"{statistics.mean(a) / 1e6:.1f} ({', '.join(kernel_ops[k])})" if a else "-"
            f.write(f"| {k} | {fetch[k]:.0f} | {write[k]:.0f} | {traffic[k] / 1e6:.1f} | {alg} | "
                    f"{ratio} |\n")
        for op, ks in OP_KERNELS.items():
            if all(k in traffic for k in ks) and op in CASES:
                tot = sum(traffic[k] for k in ks)
                f.write(f"\n{op}: its kernels move {tot / 1e6:.1f} MB in all ("
                        + " + ".join(f"{k} {traffic[k] / 1e6:.1f}" for k in ks)
                        + f"), {tot / CASES[op].algo_bytes:.3f} x the op's "
                        f"{CASES[op].algo_bytes / 1e6:.1f} MB of algorithmic bytes.\n")
    print(f"[bench] wrote profiles/ summaries from {out_dir}", file=sys.stderr)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--op", default=None, help="time only this op")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="time every op with eager launches")
    ap.add_argument("--graph", action="store_true",
                    help="time every op with a HIP graph replay")
    ap.add_argument("--floors", action="store_true",
                    help="only time the launch floor (empty kernel) and plain copies moving "
                         "the bytes of every small (graph-timed) op, and print them as JSON")
    ap.add_argument("--summarize-profile", metavar="OUT",
                    help="summarise the rocprofv3 output of PROFILE_COMMANDS under OUT into "
                         "profiles/ (no GPU needed)")
    ap.add_argument("--copy-bytes", type=int, default=0, metavar="B",
                    help="only time a plain device copy moving B bytes (B/2 read, B/2 "
                         "written), eagerly, rotated past the Infinity Cache like the ops, "
                         "and print it as JSON (a same-traffic reference for counter runs)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run plain 256 MiB device copies (the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.summarize_profile:
        summarize_profile(args.summarize_profile)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "these ops are per-rank kernels with no collectives, so run it "
              "with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration(dev, args.steps)
        return
    if args.copy_bytes:
        c = CopyFloorCase(args.copy_bytes)
        us = time_gpu(c, dev, args.steps, args.warmup, True) * 1e3
        print(json.dumps({"copy_bytes": c.algo_bytes, "timing": "eager", "us_per_call": round(us, 2),
                          "GB/s": round(c.algo_bytes / (us * 1e-6) / 1e9, 1)}))
        return
    if args.floors:
        small = [c for c in CASES.values() if c.timing == "graph"]
        fl = floors(dev, args.steps, args.warmup, sorted({c.algo_bytes for c in small}))
        fl["ops"] = {c.name: c.algo_bytes for c in small}
        print(json.dumps({"floors": fl}))
        return
    names = [args.op] if args.op else list(CASES)
    headline = args.op or HEADLINE
    ops = {}
    for name in names:
        case = CASES[name]()
        eager = args.eager or (case.timing == "eager" and not args.graph)
        ms = time_gpu(case, dev, args.steps, args.warmup, eager)
        gbs = case.algo_bytes / (ms * 1e-3) / 1e9
        ops[name] = {
            "config": case.config,
            "kernel": case.kernel,
            "timing": "eager" if eager else "graph",
            "us_per_call": round(ms * 1e3, 2),
            "algo_bytes": case.algo_bytes,
            "GB/s": round(gbs, 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)},
        }
        flops = getattr(case, "algo_flops", 0)
        if flops:
            tfs = flops / (ms * 1e-3) / 1e12
            ops[name]["tokens/s"] = round(case.tokens / (ms * 1e-3))
            ops[name]["algo_flops"] = flops
            ops[name]["mfma_roofline"] = {
                "bound": "mfma", "achieved": round(tfs, 2), "peak": MFMA_BF16_TFS,
                "unit": "TFLOP/s", "frac": round(tfs / MFMA_BF16_TFS, 4)}
            # Which floor is higher: HBM bytes at 8 TB/s or FLOPs at 2.5 PFLOP/s.
            t_hbm = case.algo_bytes / (HBM_PEAK_GBS * 1e9)
            t_mfma = flops / (MFMA_BF16_TFS * 1e12)
            ops[name]["bound"] = "hbm" if t_hbm >= t_mfma else "mfma"
            ops[name]["frac_of_bound"] = round(max(t_hbm, t_mfma) / (ms * 1e-3), 4)
        if not eager:
            # The same bytes through a plain copy kernel in the same harness:
            # how far this small op is from what its traffic allows here.
            cus = time_gpu(CopyFloorCase(case.algo_bytes), dev, args.steps, args.warmup,
                           False) * 1e3
            ops[name]["same_traffic_copy_us"] = round(cus, 2)
            ops[name]["vs_copy"] = round(ms * 1e3 / cus, 3)
        tail = getattr(case, "tail_floor", None)
        if tail:
            # The op's strided access pattern alone, without its loads of
            # other operands or its arithmetic.
            tus = time_gpu(TailFloorCase(*tail), dev, args.steps, args.warmup, False) * 1e3
            ops[name]["strided_tail_floor_us"] = round(tus, 2)
            ops[name]["vs_strided_tail_floor"] = round(ms * 1e3 / tus, 3)
        if hasattr(case, "stage_sets"):
            # Each stage alone, against the roofline of its own inputs and
            # outputs (the stage API keeps its intermediates in HBM).
            st_ms = time_stages(case, dev, args.steps, args.warmup)
            stages = []
            for (entry, kern, io), sm in zip(case.stage_io(), st_ms):
                sg = io / (sm * 1e-3) / 1e9
                stages.append({"entry_point": entry, "kernel": kern, "us_per_call": round(sm * 1e3, 2),
                               "own_io_bytes": io, "GB/s": round(sg, 1),
                               "frac_of_own_io_roofline": round(sg / HBM_PEAK_GBS, 4)})
                print(f"[bench]   stage {entry}: {sm*1e3:.2f} us, {io/1e6:.1f} MB own I/O, "
                      f"{sg / HBM_PEAK_GBS:.1%} of peak", file=sys.stderr, flush=True)
            ops[name]["stages"] = stages
            # The same access pattern as a plain copy: [T, H, 128] bf16 moved
            # by (chunk, head) tiles.
            tile = TileFloorCase(case.T, case.HV, 256)
            tus = time_gpu(tile, dev, args.steps, args.warmup, False) * 1e3
            tgb = tile.algo_bytes / (tus * 1e-6) / 1e9
            ops[name]["tile_copy_floor"] = {"config": tile.config, "us": round(tus, 2),
                                            "GB/s": round(tgb, 1)}
            for st in stages:
                st["frac_of_tile_copy"] = round(st["GB/s"] / tgb, 4)
            print(f"[bench]   tile-copy floor ({tile.config}): {tus:.2f} us, {tgb:.0f} GB/s",
                  file=sys.stderr, flush=True)
        print(f"[bench] {name}: {ms*1e3:.2f} us/call, {gbs:.0f} GB/s "
              f"({gbs / HBM_PEAK_GBS:.1%} of peak)"
              + (f", {ops[name]['tokens/s']:.3g} tokens/s, "
                 f"{ops[name]['mfma_roofline']['achieved']} TFLOP/s" if flops else ""),
              file=sys.stderr, flush=True)
    head = ops[headline]
    case = CASES[headline]()
    cpu = None
    if not args.no_cpu:
        # The CPU restatement of each op's reference on the same inputs, on
        # this host's cores, after every GPU measurement.
        for name in names:
            c = CASES[name]()
            line = cpu_line(c, ops[name]["us_per_call"])
            if line is None and name == GdnChunkStagedCase.name and \
                    GdnChunkCase.name in ops and "cpu_baseline" in ops[GdnChunkCase.name]:
                line = dict(ops[GdnChunkCase.name]["cpu_baseline"],
                            sample="the gdn_chunk_prefill line's CPU run (same workload)")
                line["gpu_speedup"] = round(line["ms_per_call"] * 1e3 / ops[name]["us_per_call"], 1)
            if line is None and name == GdnChunkStagedCase.name:
                c = GdnChunkCase()
                line = cpu_line(c, ops[name]["us_per_call"])
            if line is not None:
                ops[name]["cpu_baseline"] = line
            del c
        cpu = ops[headline].get("cpu_baseline")
    traffic = measured_traffic(case)
    # Every op's dominant kernel carries its counted HBM bytes per dispatch
    # too (null, with a warning, when its source changed since the counters
    # were taken).
    for name in names:
        ops[name]["roofline"]["traffic"] = measured_traffic(CASES[name])
    line = {
        "metric": "achieved HBM GB/s (% of peak) per op; chunked GDN prefill tokens/s",
        "value": head["GB/s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": SETTLE_S,
        "ms_per_step": round(head["us_per_call"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded torch.randn inputs of the BASELINE.json config",
        "config": {"workload": case.config, "op": headline},
        "roofline": dict(head["roofline"], traffic=traffic),
        "cpu_baseline": cpu,
        "ops": ops,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
