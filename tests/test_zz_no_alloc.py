"""xk_gdn_chunk_fwd_noalloc (the chunked gated delta rule with its workspace
in the library's static device buffer) against xk_gdn_chunk_fwd with a
caller-allocated workspace, through the C-ABI: two calls in a row, the second
on a smaller input (so the buffer holds the first call's records), each
bit-identical to the workspace entry point, which shares its kernels."""
import ctypes

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _inputs(lens, H, HV, seed):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    q = torch.randn(1, T, H, 128, generator=g).bfloat16()
    k = torch.randn(1, T, H, 128, generator=g).bfloat16()
    v = torch.randn(1, T, HV, 128, generator=g).bfloat16()
    gate = -F.softplus(torch.randn(1, T, HV, generator=g))
    beta = torch.sigmoid(torch.randn(1, T, HV, generator=g)).bfloat16()
    h0 = torch.randn(len(lens), HV, 128, 128, generator=g) * 0.05
    return q, k, v, gate, beta, h0, cu


def _noalloc(dev, q, k, v, gate, beta, h0, cu, H, HV):
    from torch_npu_ops_amd import _lib
    T, N = q.shape[1], cu.numel() - 1
    o = torch.empty(1, T, HV, 128, dtype=torch.bfloat16, device=dev)
    fin = torch.empty(N, HV, 128, 128, dtype=torch.float32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    st = _lib.lib().xk_gdn_chunk_fwd_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.XK_BF16, gate.data_ptr(), _lib.XK_F32,
        beta.data_ptr(), _lib.XK_BF16, o.data_ptr(), h0.data_ptr(), fin.data_ptr(),
        cu.data_ptr(), _lib.XK_I32, N, T, H, HV, 128, 128, 128 ** -0.5, 1, stream)
    assert st == _lib.XK_OK, _lib.status_string(st)
    return o, fin


def test_noalloc_matches_workspace_entry_point_twice(dev):
    from torch_npu_ops_amd import ops
    cases = [([900, 1, 2300, 640], 4, 8, 1), ([300, 77], 2, 4, 2)]  # second is smaller
    for lens, H, HV, seed in cases:
        print(f"noalloc case lens={lens} H={H} HV={HV}", flush=True)
        t = [x.to(dev) for x in _inputs(lens, H, HV, seed)]
        o1, f1 = _noalloc(dev, *t, H, HV)
        q, k, v, gate, beta, h0, cu = t
        o2, f2 = ops.npu_chunk_gated_delta_rule(q, k, v, gate, beta, None, h0, True, cu,
                                                False, True)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2)
        assert torch.equal(f1, f2)


_CAPTURE_CHILD = r"""
import ctypes, sys
import torch
import torch.nn.functional as F
sys.path.insert(0, sys.argv[1])
from torch_npu_ops_amd import _lib, ops
dev = torch.device("cuda:0")
g = torch.Generator().manual_seed(3)
lens, H, HV = [700, 33, 1500], 2, 4
T, N = sum(lens), len(lens)
cu = torch.zeros(N + 1, dtype=torch.int32)
cu[1:] = torch.cumsum(torch.tensor(lens), 0)
q = torch.randn(1, T, H, 128, generator=g).bfloat16().to(dev)
k = torch.randn(1, T, H, 128, generator=g).bfloat16().to(dev)
v = torch.randn(1, T, HV, 128, generator=g).bfloat16().to(dev)
gate = (-F.softplus(torch.randn(1, T, HV, generator=g))).to(dev)
beta = torch.sigmoid(torch.randn(1, T, HV, generator=g)).bfloat16().to(dev)
h0 = (torch.randn(N, HV, 128, 128, generator=g) * 0.05).to(dev)
cu = cu.to(dev)
o = torch.zeros(1, T, HV, 128, dtype=torch.bfloat16, device=dev)
fin = torch.zeros(N, HV, 128, 128, dtype=torch.float32, device=dev)
lib = _lib.lib()
torch.cuda.synchronize()
status = []
graph = torch.cuda.CUDAGraph()
print("capturing the first noalloc call of this process", flush=True)
with torch.cuda.graph(graph):
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    status.append(lib.xk_gdn_chunk_fwd_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.XK_BF16, gate.data_ptr(), _lib.XK_F32,
        beta.data_ptr(), _lib.XK_BF16, o.data_ptr(), h0.data_ptr(), fin.data_ptr(),
        cu.data_ptr(), _lib.XK_I32, N, T, H, HV, 128, 128, 128 ** -0.5, 1, stream))
assert status == [_lib.XK_OK], _lib.status_string(status[0])
o_ref, f_ref = ops.npu_chunk_gated_delta_rule(q, k, v, gate, beta, None, h0, True, cu, False, True)
torch.cuda.synchronize()
for i in range(3):
    o.zero_()
    fin.zero_()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref), f"replay {i}: o differs"
    assert torch.equal(fin, f_ref), f"replay {i}: final state differs"
    print(f"replay {i} bit-identical", flush=True)
print("ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(dev):
    """In a fresh process, the first call of the entry point (which looks up
    the device address of its static buffer) happens while a HIP graph is
    being captured; every replay of the graph then matches the workspace
    entry point bit for bit."""
    import os
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, repo], capture_output=True,
                       text=True, timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("ok")
