"""Build recipes for the native parts of torch_npu_ops_amd.

* ``libxk.so`` -- every HIP kernel plus the C-ABI of ``include/xk_ops.h``,
  compiled by hipcc for gfx950 only.  No torch dependency.
* ``_torch_api*.so`` -- the C++ drop-in layer (the reference's torch_api
  signatures) linked against libtorch and libxk.so, with a pybind module for
  tests.

Both land in-tree next to this file so that they travel with the repository
snapshot.  Objects go to ``torch_npu_ops_amd/_build/``.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libxk.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32
# (some forms have given silently wrong results on these boxes).
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wno-unused-result",
    f"-I{INCLUDE_DIR}",
    f"-I{CSRC_DIR}",
]


# Per-source extra hipcc flags (none at present).
EXTRA_FLAGS: dict[str, list[str]] = {}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature;
    # that line is expected and filtered.
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def hip_sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC_DIR, "*.hip")))


def build_lib(jobs: int | None = None, verbose: bool = True) -> str:
    """Compile every csrc/*.hip for gfx950 and link libxk.so."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = hip_sources()
    objs = [os.path.join(BUILD_DIR, os.path.basename(s) + ".o") for s in srcs]
    jobs = jobs or min(8, os.cpu_count() or 4)

    def compile_one(pair):
        src, obj = pair
        _run([HIPCC, *HIP_FLAGS, *EXTRA_FLAGS.get(os.path.basename(src), []), "-c", src,
              "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj in ex.map(compile_one, zip(srcs, objs)):
            if verbose:
                print(f"[xk build] compiled {os.path.basename(obj)}", flush=True)
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[xk build] linked {LIB_PATH}", flush=True)
    return LIB_PATH


MEASURE_DIR = os.path.join(PKG_DIR, "measure")
MEASURE_LIB_PATH = os.path.join(PKG_DIR, "libxk_measure.so")


def build_measure_lib(verbose: bool = True) -> str:
    """libxk_measure.so: bench.py's reference kernels (empty kernel, plain
    copy).  Measurement only; not part of the C-ABI."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(MEASURE_DIR, "*.hip")))
    objs = []
    for src in srcs:
        obj = os.path.join(BUILD_DIR, "measure_" + os.path.basename(src) + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
        objs.append(obj)
    tmp = MEASURE_LIB_PATH + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp])
    os.replace(tmp, MEASURE_LIB_PATH)
    if verbose:
        print(f"[xk build] linked {MEASURE_LIB_PATH}", flush=True)
    return MEASURE_LIB_PATH


TORCH_API_DIR = os.path.join(CSRC_DIR, "torch_api")
TORCH_API_PATH = os.path.join(PKG_DIR, "_xk_torch.so")


def torch_api_sources() -> list[str]:
    return sorted(glob.glob(os.path.join(TORCH_API_DIR, "*.cpp")))


def build_torch_api(jobs: int | None = None, verbose: bool = True) -> str:
    """Compile the C++ drop-in layer (csrc/torch_api) with g++ against the
    installed PyTorch-ROCm and link _xk_torch.so against libxk.so (found
    next to it through an $ORIGIN rpath).  Needs libxk.so built first."""
    import sysconfig

    import torch
    torch_dir = os.path.dirname(torch.__file__)
    os.makedirs(BUILD_DIR, exist_ok=True)
    cxx = os.environ.get("CXX", "g++")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    flags = [
        "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_xk_torch", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-I{os.path.join(torch_dir, 'include')}",
        f"-I{os.path.join(torch_dir, 'include', 'torch', 'csrc', 'api', 'include')}",
        "-I/opt/rocm/include", f"-I{sysconfig.get_paths()['include']}",
        f"-I{INCLUDE_DIR}", f"-I{TORCH_API_DIR}",
        "-Wno-deprecated-declarations",
    ]
    srcs = torch_api_sources()
    objs = [os.path.join(BUILD_DIR, "torch_api_" + os.path.basename(s) + ".o") for s in srcs]
    jobs = jobs or min(8, os.cpu_count() or 4)

    def compile_one(pair):
        src, obj = pair
        _run([cxx, *flags, "-c", src, "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj in ex.map(compile_one, zip(srcs, objs)):
            if verbose:
                print(f"[xk build] compiled {os.path.basename(obj)}", flush=True)
    tmp = TORCH_API_PATH + ".tmp"
    _run([cxx, "-shared", *objs, "-o", tmp,
          f"-L{os.path.join(torch_dir, 'lib')}", "-L/opt/rocm/lib",
          f"-L{PKG_DIR}", "-lxk", "-Wl,-rpath,$ORIGIN",
          "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_hip", "-ltorch_python",
          "-lamdhip64"])
    os.replace(tmp, TORCH_API_PATH)
    if verbose:
        print(f"[xk build] linked {TORCH_API_PATH}", flush=True)
    return TORCH_API_PATH


CONSUMER_SRC = os.path.join(REPO_DIR, "tests", "cpp", "api_consumer.cpp")
CONSUMER_PATH = os.path.join(REPO_DIR, "tests", "cpp", "xk_api_consumer")


def build_api_consumer(verbose: bool = True) -> str:
    """tests/cpp/xk_api_consumer: a C++ executable (no Python) that links the
    drop-in layer's objects (torch_api.cpp, registry.cpp, compiled by
    build_torch_api), libxk.so and libtorch, as an engine would.  Its NEEDED
    list names the torch libraries before libxk.so, so that the loader maps
    PyTorch's HIP runtime first and libxk.so binds to it by soname."""
    import torch
    torch_dir = os.path.dirname(torch.__file__)
    torch_lib = os.path.join(torch_dir, "lib")
    cxx = os.environ.get("CXX", "g++")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    obj = os.path.join(BUILD_DIR, "api_consumer.o")
    _run([cxx, "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
          f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          f"-I{os.path.join(torch_dir, 'include')}",
          f"-I{os.path.join(torch_dir, 'include', 'torch', 'csrc', 'api', 'include')}",
          "-I/opt/rocm/include", f"-I{INCLUDE_DIR}", f"-I{TORCH_API_DIR}",
          "-Wno-deprecated-declarations", "-c", CONSUMER_SRC, "-o", obj])
    api_objs = [os.path.join(BUILD_DIR, "torch_api_" + n + ".o")
                for n in ("torch_api.cpp", "registry.cpp")]
    rel = os.path.relpath(PKG_DIR, os.path.dirname(CONSUMER_PATH))
    tmp = CONSUMER_PATH + ".tmp"
    _run([cxx, obj, *api_objs, "-o", tmp,
          f"-L{torch_lib}", f"-L{PKG_DIR}",
          f"-Wl,-rpath,{torch_lib}", f"-Wl,-rpath,$ORIGIN/{rel}",
          "-Wl,--no-as-needed", "-ltorch", "-ltorch_cpu", "-lc10", "-lc10_hip", "-ltorch_hip",
          "-lxk", "-Wl,--as-needed"])
    os.replace(tmp, CONSUMER_PATH)
    if verbose:
        print(f"[xk build] linked {CONSUMER_PATH}", flush=True)
    return CONSUMER_PATH


def build_all(verbose: bool = True) -> None:
    build_lib(verbose=verbose)
    build_torch_api(verbose=verbose)
    build_api_consumer(verbose=verbose)
    build_measure_lib(verbose=verbose)


def clean() -> None:
    shutil.rmtree(BUILD_DIR, ignore_errors=True)


if __name__ == "__main__":
    build_all()
