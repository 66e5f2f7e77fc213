#!/usr/bin/env python3
"""Benchmark of the xLLM op set on one MI355X.

    python bench.py [--steps K] [--warmup W] [--op NAME] [--no-cpu]

One step = one call of the op on its BASELINE config with inputs already
resident in HBM.  Rank 0 prints ONE JSON line:
  value       achieved GB/s of the headline op (algorithmic bytes / time)
  roofline    achieved / peak for the dominant kernel, from per-launch HIP
              events recorded on the stream the kernels run on
  cpu_baseline the oracle (CPU restatement of the reference) on host cores
  ops         every op's line (config, us/call, GB/s or tokens/s, roofline)
Inputs rotate over several buffer sets whose total exceeds the 256 MB
Infinity Cache so that timings see HBM, not the cache.
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
ROTATE_BYTES = 1 << 30  # >= 1 GiB of distinct buffers per op
CPU_THREADS = min(16, os.cpu_count() or 1)

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


# ---------------------------------------------------------------------------
# Op cases.  Each builds seeded inputs (on the CPU, copied to the GPU),
# returns a GPU closure per buffer set, the algorithmic bytes per call and a
# CPU closure for the baseline.
# ---------------------------------------------------------------------------
class Case:
    name = ""
    config = ""
    dtype = "bf16"
    algo_bytes = 0
    kernel = ""

    def sets(self, dev, n):  # -> list of callables
        raise NotImplementedError

    def cpu(self):  # -> (callable, sample description, scale to one call)
        raise NotImplementedError


def _randn(shape, gen, dtype, scale=1.0, shift=0.0):
    return (torch.randn(shape, generator=gen) * scale + shift).to(dtype)


class LayerNormCase(Case):
    name = "layer_norm_fwd"
    config = ("config 2a: layer_norm_fwd bf16 x[16384,4096], group_size 4096, "
              "affine w~N(1,0.1) b~N(0,0.1), eps 1e-5, outputs y + fp32 mean/rstd")
    kernel = "layer_norm_fwd_kernel"
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
        from torch_npu_ops_amd.ops import _stream
        lib = _lib.lib()
        w, b = self.w.to(dev), self.b.to(dev)
        out = []
        for _ in range(n):
            x = self.x.to(dev)
            y = torch.empty_like(x)
            mean = torch.empty(self.M, dtype=torch.float32, device=dev)
            rstd = torch.empty(self.M, dtype=torch.float32, device=dev)
            s = _stream(x)

            def run(x=x, y=y, mean=mean, rstd=rstd, s=s):
                st = lib.xk_layer_norm_fwd(
                    x.data_ptr(), self.N, y.data_ptr(), self.N, w.data_ptr(),
                    b.data_ptr(), None, 0, mean.data_ptr(), rstd.data_ptr(),
                    self.M, self.N, self.N, 1e-5, 1, 0, _lib.XK_BF16,
                    _lib.XK_BF16, s)
                if st:
                    raise RuntimeError(_lib.status_string(st))
            out.append(run)
        return out

    def cpu(self):
        from oracle import norm as on
        x, w, b = self.x, self.w, self.b

        def run():
            on.layer_norm_fwd(x, w, b, 1e-5)
        return run, "full config 2a (16384x4096), fp32 math on bf16 input", 1.0


class GemmaCase(Case):
    name = "gemma_rms_norm"
    config = ("config 2b: Gemma RMSNorm bf16 x[16384,4096], gamma~N(1,0.1) "
              "applied as (1+gamma), eps 1e-5, outputs y + fp32 rstd")
    kernel = "layer_norm_fwd_kernel"
    M, N = 16384, 4096
    algo_bytes = M * N * 2 * 2 + M * 4 + N * 2

    def __init__(self):
        g = torch.Generator().manual_seed(0)
        self.x = _randn((self.M, self.N), g, torch.bfloat16)
        self.gamma = _randn((self.N,), g, torch.bfloat16, 0.1, 1.0)

    def sets(self, dev, n):
        from torch_npu_ops_amd import _lib
        from torch_npu_ops_amd.ops import _stream
        lib = _lib.lib()
        gamma = self.gamma.to(dev)
        out = []
        for _ in range(n):
            x = self.x.to(dev)
            y = torch.empty_like(x)
            rstd = torch.empty(self.M, dtype=torch.float32, device=dev)
            s = _stream(x)

            def run(x=x, y=y, rstd=rstd, s=s):
                st = lib.xk_gemma_rms_norm(
                    x.data_ptr(), self.N, y.data_ptr(), self.N,
                    gamma.data_ptr(), rstd.data_ptr(), self.M, self.N, 1e-5,
                    _lib.XK_BF16, _lib.XK_BF16, s)
                if st:
                    raise RuntimeError(_lib.status_string(st))
            out.append(run)
        return out

    def cpu(self):
        from oracle import norm as on
        x, gamma = self.x, self.gamma

        def run():
            on.gemma_rms_norm(x, gamma, 1e-5)
        return run, "full config 2b (16384x4096), fp32 math on bf16 input", 1.0


CASES = {c.name: c for c in (LayerNormCase, GemmaCase)}
HEADLINE = "layer_norm_fwd"


# ---------------------------------------------------------------------------
# Timing
# ---------------------------------------------------------------------------
def time_gpu(case: Case, dev, steps: int, warmup: int):
    per_set = max(case.algo_bytes, 1)
    nsets = max(2, min(16, -(-ROTATE_BYTES // per_set)))
    runs = case.sets(dev, nsets)
    for i in range(warmup):
        runs[i % nsets]()
    torch.cuda.synchronize()
    # Whole-region time (ms_per_step) ...
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        runs[i % nsets]()
    t1.record()
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / steps
    # ... and per-launch event pairs for the kernel's own duration.  The
    # kernels run on torch's current stream, where these events are recorded.
    evs = [(torch.cuda.Event(enable_timing=True),
            torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i, (a, b) in enumerate(evs):
        a.record()
        runs[i % nsets]()
        b.record()
    torch.cuda.synchronize()
    launch_ms = [a.elapsed_time(b) for a, b in evs]
    del runs
    torch.cuda.empty_cache()
    return ms_per_step, statistics.mean(launch_ms), statistics.median(launch_ms)


def time_cpu(case: Case):
    torch.set_num_threads(CPU_THREADS)
    run, sample, scale = case.cpu()
    run()  # warm-up
    ts = []
    budget_end = time.perf_counter() + 20.0
    while len(ts) < 3 or (time.perf_counter() < budget_end and len(ts) < 5):
        t = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t)
        if time.perf_counter() > budget_end and len(ts) >= 1:
            break
    sec = statistics.median(ts) * scale
    return sec, sample, len(ts)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--op", default=None, help="time only this op")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "the ops are per-rank kernels with no collectives, so run it "
              "with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    names = [args.op] if args.op else list(CASES)
    headline = args.op or HEADLINE
    ops = {}
    for name in names:
        case = CASES[name]()
        ms, launch_mean, launch_med = time_gpu(case, dev, args.steps, args.warmup)
        gbs = case.algo_bytes / (ms * 1e-3) / 1e9
        kgbs = case.algo_bytes / (launch_mean * 1e-3) / 1e9
        ops[name] = {
            "config": case.config,
            "us_per_call": round(ms * 1e3, 2),
            "kernel_us_mean": round(launch_mean * 1e3, 2),
            "kernel_us_median": round(launch_med * 1e3, 2),
            "algo_bytes": case.algo_bytes,
            "GB/s": round(gbs, 1),
            "roofline": {"bound": "hbm", "achieved": round(kgbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(kgbs / HBM_PEAK_GBS, 4)},
        }
        print(f"[bench] {name}: {ms*1e3:.1f} us/call, {gbs:.0f} GB/s", file=sys.stderr,
              flush=True)
    head = ops[headline]
    case = CASES[headline]()
    cpu = None
    if not args.no_cpu:
        sec, sample, nrun = time_cpu(case)
        cpu = {"value": round(case.algo_bytes / sec / 1e9, 2), "unit": "GB/s",
               "cores": CPU_THREADS, "kind": "port",
               "sample": f"{sample}; median of {nrun} runs, {sec*1e3:.1f} ms/call"}
        print(f"[bench] cpu baseline {headline}: {sec*1e3:.1f} ms/call", file=sys.stderr)
    line = {
        "metric": "achieved HBM GB/s (% of peak) per op; chunked GDN prefill tokens/s",
        "value": head["GB/s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_call"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded torch.randn inputs of the BASELINE.json config",
        "config": {"workload": case.config, "op": headline},
        "roofline": dict(head["roofline"], traffic=None),
        "cpu_baseline": cpu,
        "ops": ops,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
