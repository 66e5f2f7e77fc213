"""ctypes binding of libxk.so (the C-ABI declared in include/xk_ops.h).

torch is imported before the library is opened: libxk.so needs
``libamdhip64.so.7`` and must bind to the HIP runtime torch already loaded
(same SONAME), not to a second copy, so that torch's streams and device
pointers are valid in the kernels' runtime.

There is no fallback: if libxk.so is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import os
import re

import torch  # noqa: F401  (must precede the dlopen, see module doc)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libxk.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "xk_ops.h")

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
INT = ctypes.c_int
F32 = ctypes.c_float
SZ = ctypes.c_size_t

# xk_dtype values (include/xk_ops.h)
XK_F32, XK_BF16, XK_F16, XK_I32, XK_I64 = 0, 1, 2, 3, 4
XK_OK, XK_ERR_INVALID, XK_ERR_UNSUPPORTED, XK_ERR_WORKSPACE, XK_ERR_SCRATCH = 0, -1, -2, -3, -4

# Argument lists, in declaration order of include/xk_ops.h.
SIGNATURES: dict[str, tuple[list, object]] = {
    "xk_version": ([], ctypes.c_char_p),
    "xk_status_string": ([INT], ctypes.c_char_p),
    "xk_layer_norm_fwd": (
        [P, I64, P, I64, P, P, P, I64, P, P, I64, I64, I64, F32, INT, INT, INT,
         INT, P], INT),
    "xk_gemma_rms_norm": ([P, I64, P, I64, P, P, I64, I64, F32, INT, INT, P],
                          INT),
    "xk_l2norm_last_dim": ([P, P, I64, I64, F32, INT, INT, P], INT),
    "xk_split_rmsnorm_rope": (
        [P, I64, I64, P, P, I64, P, INT, P, P, P, P, P, P, P, P, INT, I64, I64,
         I64, F32, INT, P], INT),
    "xk_rope_inplace": ([P, I64, I64, I64, I64, P, P, I64, I64, INT, INT, P], INT),
    "xk_causal_conv1d_update": (
        [P, I64, I64, I64, P, I64, I64, I64, P, I64, I64, P, INT, P, I32, I64,
         P, I64, I64, I64, I64, I64, I64, I64, I64, INT, INT, P], INT),
    "xk_causal_conv1d_varlen": (
        [P, I64, I64, P, I64, P, I64, I64, I64, I64, I64, P, I64, I64, P, INT,
         P, I64, P, I64, INT, P, P, P, I64, I64, I64, INT, INT, I32, INT, P],
        INT),
    "xk_gdn_recurrent": (
        [P, P, P, INT, P, INT, P, INT, P, P, I64, P, I64, I64, P, INT, P, I64,
         I64, P, I64, I64, I64, I64, I64, I64, F32, INT, INT, P], INT),
    "xk_fused_gdn_gating": ([P, P, P, P, P, P, I64, I64, F32, F32, INT, P], INT),
    "xk_gdn_sigmoid_gating_update": (
        [P, P, P, F32, F32, P, P, P, P, INT, P, P, I64, I64, P, P, I64, I64, I64,
         I64, I64, F32, INT, INT, P], INT),
    "xk_fused_qkvzba_split_reshape_cat": (
        [P, I64, P, I64, P, P, P, P, I64, I64, I64, I64, I64, INT, INT, P], INT),
    "xk_gdn_conv_decode": (
        [P, I64, P, I64, I64, I64, I64, I64, P, I64, I64, P, INT, I64, P, I32,
         P, INT, P, INT, P, I64, I64, P, P, I64, I64, I64, I64, I64, F32, INT,
         INT, P], INT),
    "xk_gdn_conv_gating_decode": (
        [P, I64, P, I64, I64, I64, I64, I64, P, I64, I64, P, INT, I64, P, I32,
         P, P, P, P, INT, F32, F32, P, I64, I64, P, P, I64, I64, I64, I64, I64,
         F32, INT, INT, P], INT),
    "xk_gdn_chunk_workspace_bytes": ([I64, I64, I64], I64),
    "xk_gdn_chunk_fwd": (
        [P, P, P, INT, P, INT, P, INT, P, P, P, P, INT, I64, I64, I64, I64, I64,
         I64, F32, INT, P, SZ, P], INT),
    "xk_gdn_chunk_fwd_noalloc": (
        [P, P, P, INT, P, INT, P, INT, P, P, P, P, INT, I64, I64, I64, I64, I64,
         I64, F32, INT, P], INT),
    "xk_gdn_stage_workspace_bytes": ([I64], I64),
    "xk_chunk_local_cumsum": ([P, INT, P, I64, I64, P, INT, I64, I64, P], INT),
    "xk_chunk_scaled_dot_kkt": (
        [P, INT, P, INT, P, P, I64, I64, I64, I64, P, INT, I64, P, SZ, P], INT),
    "xk_solve_tril": ([P, P, INT, I64, I64, P, INT, I64, P, SZ, P], INT),
    "xk_recompute_w_u": (
        [P, P, INT, P, INT, P, P, INT, P, P, I64, I64, I64, I64, I64, P, INT,
         I64, P, SZ, P], INT),
    "xk_chunk_fwd_h": (
        [P, P, P, INT, P, P, P, I64, P, P, I64, I64, I64, I64, I64, P, INT, I64,
         P, SZ, P], INT),
    "xk_chunk_fwd_o": (
        [P, P, P, P, I64, INT, P, P, F32, I64, I64, I64, I64, I64, P, INT, I64,
         P, SZ, P], INT),
}

_LIB = None


def declared_symbols() -> list[str]:
    """Function names declared in include/xk_ops.h."""
    text = open(HEADER_PATH).read()
    return re.findall(r"^\s*(?:const\s+)?(?:int|int64_t|const char\*|size_t)\s*\*?\s*(xk_\w+)\s*\(",
                      text, flags=re.M)


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = handle
    return _LIB


def status_string(status: int) -> str:
    return lib().xk_status_string(status).decode()


def check(status: int, what: str) -> None:
    if status != XK_OK:
        raise RuntimeError(f"{what} failed: {status_string(status)} ({status})")
