"""CPU checks of the C-ABI library: it loads, exports every symbol that
include/xk_ops.h declares, and rejects bad arguments before touching a GPU."""
import ctypes

import pytest

from torch_npu_ops_amd import _lib


def test_header_declares_functions():
    names = _lib.declared_symbols()
    assert "xk_layer_norm_fwd" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    handle = _lib.lib()
    missing = [n for n in _lib.declared_symbols() if not hasattr(handle, n)]
    assert not missing, f"libxk.so lacks {missing}"


def test_every_declared_symbol_has_a_ctypes_signature():
    missing = [n for n in _lib.declared_symbols() if n not in _lib.SIGNATURES]
    assert not missing


def test_version_and_status_strings():
    assert b"gfx950" in _lib.lib().xk_version()
    assert _lib.status_string(_lib.XK_ERR_INVALID) == "invalid argument"
    assert _lib.status_string(_lib.XK_ERR_WORKSPACE).startswith("workspace")


def test_layer_norm_rejects_bad_group_size_without_gpu():
    st = _lib.lib().xk_layer_norm_fwd(None, 0, None, 0, None, None, None, 0,
                                      None, None, 4, 100, 33, 1e-5, 1, 0,
                                      _lib.XK_BF16, _lib.XK_BF16, None)
    assert st == _lib.XK_ERR_INVALID


def test_layer_norm_rejects_integer_dtype_without_gpu():
    st = _lib.lib().xk_layer_norm_fwd(None, 0, None, 0, None, None, None, 0,
                                      None, None, 4, 128, 128, 1e-5, 1, 0,
                                      _lib.XK_I32, _lib.XK_BF16, None)
    assert st == _lib.XK_ERR_UNSUPPORTED


def test_empty_input_is_a_no_op_without_gpu():
    st = _lib.lib().xk_layer_norm_fwd(None, 0, None, 0, None, None, None, 0,
                                      None, None, 0, 128, 128, 1e-5, 1, 0,
                                      _lib.XK_BF16, _lib.XK_BF16, None)
    assert st == _lib.XK_OK


def test_noalloc_chunk_rejects_problems_beyond_its_scratch_without_gpu():
    # 64 MiB of static scratch: 100k tokens at 32 v-heads need ~2 GB of
    # records, so the call is refused before any GPU work.
    lib = _lib.lib()
    need = lib.xk_gdn_chunk_workspace_bytes(100_000, 8, 32)
    assert need > 64 << 20
    st = lib.xk_gdn_chunk_fwd_noalloc(
        None, None, None, _lib.XK_BF16, None, _lib.XK_F32, None, _lib.XK_BF16, None, None,
        None, None, _lib.XK_I32, 8, 100_000, 16, 32, 128, 128, 0.1, 1, None)
    assert st == _lib.XK_ERR_SCRATCH
    assert "static scratch" in _lib.status_string(st)
    st = lib.xk_gdn_chunk_fwd_noalloc(
        None, None, None, _lib.XK_BF16, None, _lib.XK_F32, None, _lib.XK_BF16, None, None,
        None, None, _lib.XK_I32, -1, 100, 16, 32, 128, 128, 0.1, 1, None)
    assert st == _lib.XK_ERR_INVALID
