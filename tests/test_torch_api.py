"""The C++ drop-in layer (csrc/torch_api, module _xk_torch) on the CPU: it
loads, its registry / operation-factory shims map the reference's kernel
names onto the C-ABI, and its validation raises like the reference wrappers
before anything touches a GPU."""
import ctypes

import pytest
import torch


@pytest.fixture(scope="module")
def xt():
    from torch_npu_ops_amd import _xk_torch
    return _xk_torch


def test_registry_maps_reference_names_to_entry_points(xt):
    from torch_npu_ops_amd import _lib
    lib = _lib.lib()
    pairs = {
        "layer_norm_fwd_kernel_fast_rms_bf16_z_nobias_nomask": "xk_layer_norm_fwd",
        "fused_recurrent_gated_delta_rule_spec_fwd_kernel": "xk_gdn_recurrent",
        "chunk_gated_delta_rule_fwd_kernel_h_blockdim64": "xk_chunk_fwd_h",
        "merge_16x16_to_64x64_inverse_kernel": "xk_solve_tril",
        "_causal_conv1d_update_kernel_npu_tiled_v2": "xk_causal_conv1d_varlen",
        "split_rmsnorm_rope_kernel": "xk_split_rmsnorm_rope",
        "fused_gdn_gating_decode_kernel": "xk_fused_gdn_gating",
        "fused_sigmoid_gating_delta_rule_update_kernel": "xk_gdn_sigmoid_gating_update",
        "fused_qkvzba_split_reshape_cat_gqa_r3_kernel": "xk_fused_qkvzba_split_reshape_cat",
        "rope_inplace_kernel": "xk_rope_inplace",
    }
    for name, sym in pairs.items():
        assert xt.registry_register(name, "/path/ignored.npubin")
        assert xt.registry_stub(name) == ctypes.cast(getattr(lib, sym), ctypes.c_void_p).value
    # kernels outside the op set are not registered
    assert not xt.registry_register("_causal_conv1d_fwd_kernel", "")
    assert xt.registry_stub("_causal_conv1d_update_kernel_no_cache_len") == 0


def test_factory_names_and_status_forwarding(xt):
    assert xt.factory_kernel_name("layer_norm_fwd") == "layer_norm_fwd_kernel"
    assert xt.factory_kernel_name("chunk_fwd_o") == "chunk_fwd_kernel_o"
    # execute() returns the C-ABI status of an invalid call (M < 0)
    assert xt.factory_status_of_invalid_layer_norm() == -1


def test_validation_errors_match_reference_messages(xt):
    x = torch.zeros(4, 12)
    with pytest.raises(RuntimeError, match="divisible by group_size"):
        xt.layer_norm_fwd(x, torch.ones(12), torch.zeros(12), 1e-5, None, 5)
    with pytest.raises(RuntimeError, match="head_first=false"):
        q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16)
        xt.npu_chunk_gated_delta_rule(q, q, q, torch.zeros(1, 8, 2), torch.zeros(1, 8, 2),
                                      head_first=True)
    with pytest.raises(RuntimeError, match="expects q/k/v to be bfloat16"):
        q = torch.zeros(1, 8, 2, 128)
        xt.npu_chunk_gated_delta_rule(q, q, q, torch.zeros(1, 8, 2), torch.zeros(1, 8, 2))
    with pytest.raises(RuntimeError, match="width in \\[1, 6\\]"):
        xt.npu_causal_conv1d_update_v2(torch.zeros(2, 8), torch.zeros(2, 8, 6),
                                       torch.zeros(8, 7))
    with pytest.raises(RuntimeError, match="power of two"):
        xt.npu_chunk_local_cumsum(torch.zeros(1, 8, 2), 48)


def test_cpu_tensors_are_refused(xt):
    with pytest.raises(RuntimeError, match="GPU device"):
        xt.layer_norm_fwd(torch.zeros(4, 8), torch.ones(8), torch.zeros(8), 1e-5)
    with pytest.raises(RuntimeError, match="GPU device"):
        xt.npu_ops_gemma_rms_norm(torch.zeros(4, 8), torch.ones(8), 1e-6)


def test_conv_update_query_start_loc_sentinel(xt):
    # reference :41-45 warns (TORCH_WARN, c10's log) and returns zeros(1)
    out = xt.npu_causal_conv1d_update(torch.zeros(2, 8), torch.zeros(2, 8, 3),
                                      torch.zeros(8, 4),
                                      query_start_loc=torch.tensor([0, 1, 2]))
    assert out.shape == (1,) and out.item() == 0


def test_chunk_initial_state_dtype_is_checked(xt):
    # reference npu_triton_chunk_gated_delta_rule.cpp:574-579
    q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="initial_state to be bfloat16 or float32"):
        xt.npu_chunk_gated_delta_rule(q, q, q, torch.zeros(1, 8, 2), torch.zeros(1, 8, 2),
                                      initial_state=torch.zeros(1, 2, 128, 128,
                                                                dtype=torch.float16))


def _conv_decode_args(ssm_dtype=torch.float32, conv_dtype=torch.bfloat16, ssm_shape=None):
    B, H, HV, K = 2, 1, 2, 128
    D = 2 * H * K + HV * K
    x = torch.zeros(B, D, dtype=torch.bfloat16)
    conv_state = torch.zeros(B, D, 3, dtype=conv_dtype)
    w = torch.zeros(D, 4, dtype=torch.bfloat16)
    g = torch.zeros(B, HV)
    beta = torch.zeros(B, HV, dtype=torch.bfloat16)
    ssm = torch.zeros(ssm_shape or (B, HV, K, K), dtype=ssm_dtype)
    return x, conv_state, w, g, beta, ssm, H, HV


@pytest.mark.parametrize("bad,match", [
    (dict(ssm_dtype=torch.bfloat16), "ssm_state must be float32"),
    (dict(ssm_shape=(2, 2, 128, 64)), "ssm_state must have shape"),
    (dict(conv_dtype=torch.float32), "conv_state must have mixed_qkv's dtype"),
])
def test_gdn_conv_decode_rejects_bad_state_buffers(xt, bad, match):
    # A state of another dtype or shape would be indexed past its end by the
    # kernel; both the C++ drop-in and the Python mirror refuse it first.
    from torch_npu_ops_amd import ops
    args = _conv_decode_args(**bad)
    with pytest.raises(RuntimeError, match=match):
        xt.npu_gdn_conv_decode(*args)
    with pytest.raises(ValueError, match=match):
        ops.gdn_conv_decode(*args)


def test_gdn_conv_decode_rejects_non_contiguous_state(xt):
    from torch_npu_ops_amd import ops
    x, cs, w, g, beta, _, H, HV = _conv_decode_args()
    ssm = torch.zeros(2, HV, 128, 128).transpose(2, 3)
    with pytest.raises(RuntimeError, match="contiguous within each slot"):
        xt.npu_gdn_conv_decode(x, cs, w, g, beta, ssm, H, HV)
    with pytest.raises(ValueError, match="contiguous within each slot"):
        ops.gdn_conv_decode(x, cs, w, g, beta, ssm, H, HV)


def test_operation_base_keeps_npubin_path_parameter(xt):
    # OperationBase(kernel_name, npubin_path = "") as operation_base.h:130-133
    assert xt.operation_base_paths("k", "/x/k.npubin") == ("k", "/x/k.npubin")
    assert xt.operation_base_paths("k", None) == ("k", "")
