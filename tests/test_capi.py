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
    # records, so the call is refused before any GPU work.  The pointers are
    # placeholders (aligned, never dereferenced: the entry point checks the
    # arguments, then the size, before it touches the device).
    lib = _lib.lib()
    need = lib.xk_gdn_chunk_workspace_bytes(100_000, 8, 32)
    assert need > 64 << 20
    fake = 1 << 20

    def call(N, T, H=16, HV=32, dtype=_lib.XK_BF16, ptr=fake):
        return lib.xk_gdn_chunk_fwd_noalloc(
            ptr, ptr, ptr, dtype, ptr, _lib.XK_F32, ptr, _lib.XK_BF16, ptr, None,
            None, ptr, _lib.XK_I32, N, T, H, HV, 128, 128, 0.1, 1, None)
    st = call(8, 100_000)
    assert st == _lib.XK_ERR_SCRATCH
    assert "static scratch" in _lib.status_string(st)
    # The same argument checks as xk_gdn_chunk_fwd come first.
    assert call(-1, 100) == _lib.XK_ERR_INVALID
    assert call(8, 100_000, H=3) == _lib.XK_ERR_INVALID          # HV % H != 0
    assert call(8, 100_000, dtype=_lib.XK_F32) == _lib.XK_ERR_UNSUPPORTED
    assert call(8, 100_000, ptr=None) == _lib.XK_ERR_INVALID     # NULL inputs
    assert call(0, 0, ptr=None) == _lib.XK_OK                    # no work
