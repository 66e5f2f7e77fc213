"""CPU oracle for the xLLM Triton-Ascend op set (TEST INFRASTRUCTURE ONLY).

Each module restates, in plain torch on the CPU (fp32 by default, fp64 on
request), the PyTorch / libtorch reference the upstream repository checks its
kernels against, and cites the file:line it follows.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and
only as the checker or the timed CPU baseline: nothing in the product path
(torch_npu_ops_amd/, include/) imports, links or calls it.

How each function is pinned (checks that do not retype its formula) is stated
in its docstring and exercised in tests/test_oracle_*.py.
"""
