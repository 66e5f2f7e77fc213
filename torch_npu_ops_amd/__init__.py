"""torch_npu_ops_amd: gfx950 HIP kernels for xLLM's Triton-Ascend op set.

Layers:
  include/xk_ops.h + csrc/*.hip  -> libxk.so (C-ABI, no torch)
  torch_api/                     -> C++ drop-in with the reference's
                                    torch_api signatures (_torch_api*.so)
  ops.py                         -> Python view over the C-ABI for tests,
                                    bench and smoke
"""
__version__ = "0.1.0"
