"""The C++ drop-in called from C++, as an engine calls it: tests/cpp/
xk_api_consumer links csrc/torch_api/{torch_api,registry}.cpp, libxk.so and
libtorch (no Python, no pybind), registers the kernels by name as the
reference gtests do (triton_chunk_gated_delta_rule_test.cpp:330-340) and
calls xllm::kernel::npu::layer_norm_fwd and npu_chunk_gated_delta_rule on the
committed golden inputs.  Its outputs must match the golden outputs at each
case's tolerances.
"""
import os
import subprocess
import sys

import pytest
import torch
from safetensors.torch import load_file

HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "cpp", "xk_api_consumer")
sys.path.insert(0, os.path.join(HERE, "golden"))
from cases import CASES  # noqa: E402
from make_golden import PATH  # noqa: E402


def _exe():
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built: run __graft_entry__.build() first")
    return EXE


def test_consumer_links_and_registers():
    """No GPU call: the registry accepts the reference's kernel names,
    rejects unknown ones, and the process maps exactly one HIP runtime."""
    r = subprocess.run([_exe(), "--registry"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "registry ok" in r.stdout


@pytest.mark.gpu
def test_consumer_matches_golden(tmp_path):
    out_path = str(tmp_path / "consumer_out.safetensors")
    print("running the C++ consumer on the golden inputs", flush=True)
    r = subprocess.run([_exe(), PATH, out_path], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    got = load_file(out_path)
    gold = load_file(PATH)
    checks = [("layer_norm_gated", "y"), ("gdn_chunk", "o"), ("gdn_chunk", "state")]
    assert sorted(got) == sorted(f"{c}/{k}" for c, k in checks)
    for case, key in checks:
        ref = gold[f"{case}/out/{key}"].float()
        tol = dict(CASES[case].tol[key])
        if "atol_per_rms" in tol:  # fp32 states: atol = min(1e-4, 1e-3 * RMS(reference))
            rms = ref.double().pow(2).mean().sqrt().item()
            tol["atol"] = min(tol.pop("atol_max"), tol.pop("atol_per_rms") * rms)
        torch.testing.assert_close(got[f"{case}/{key}"], ref, **tol, msg=f"{case}/{key}")
