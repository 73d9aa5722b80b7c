"""Builds ``libtokquay_amd.so`` (the gfx950 kernels and their C ABI) in place,
then the host-only CPython extension ``_native`` that links it.

Run ``python -m tokquay_amd.build``. The library is compiled straight with
``hipcc`` for gfx950 only; it has no torch dependency, so any host program can
load it through ``include/tokquay_amd.h``. ``_native`` (the batch view's
metadata builder and per-layer launcher, ``csrc/native.cpp``) is plain C++
built with the host compiler against the Python headers; it finds the kernel
library next to itself (rpath ``$ORIGIN``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
LIB_NAME = "libtokquay_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
OFFLOAD_ARCH = "gfx950"
NATIVE_SRC = os.path.join(CSRC_DIR, "native.cpp")
NATIVE_PATH = os.path.join(PKG_DIR, "_native" + sysconfig.get_config_var("EXT_SUFFIX"))
TORCH_OPS_SRC = os.path.join(CSRC_DIR, "torch_ops.cpp")
TORCH_OPS_PATH = os.path.join(PKG_DIR, "_torch_ops.so")
ROCM_INCLUDE = "/opt/rocm/include"

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed fp32 VALU ops (v_pk_*_f32) are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA sources and results in VGPRs instead of accumulator registers: the
    # prefill kernel rescales and reads its accumulators every key tile, and the
    # AGPR form paid a copy in and out for each access.
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    "-Wall",
]


def sources() -> list[str]:
    """The kernel sources (every ``*.hip`` under ``csrc``)."""
    return sorted(os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip"))


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build the kernels)")
    return path


def build(verbose: bool = False) -> str:
    """Compile every kernel source into LIB_PATH, then the ``_native`` extension and the torch
    operator library; return LIB_PATH."""
    build_kernels(verbose)
    build_native(verbose)
    build_torch_ops(verbose)
    return LIB_PATH


def build_kernels(verbose: bool = False) -> str:
    """Compile every kernel source into LIB_PATH and return that path."""
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", "-o", tmp, *sources()]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host compiler pass does not know the packed-fp32 target feature and says so; that is expected.
    noise = ("packed-fp32-ops", "not a recognized feature", "warning generated", "warnings generated")
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if ln.strip() and not any(n in ln for n in noise)]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_native(verbose: bool = False) -> str:
    """Compile ``csrc/native.cpp`` into the ``_native`` extension (links LIB_PATH) and return its path."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler (g++) found")
    tmp = NATIVE_PATH + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-missing-field-initializers",
           f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE_DIR}", "-o", tmp, NATIVE_SRC,
           f"-L{PKG_DIR}", "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN"]  # fmt: skip
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{cxx} failed ({proc.returncode}):\n{proc.stdout}{proc.stderr}")
    if verbose and (proc.stdout or proc.stderr):
        print(proc.stdout + proc.stderr, flush=True)
    os.replace(tmp, NATIVE_PATH)
    return NATIVE_PATH


def build_torch_ops(verbose: bool = False) -> str:
    """Compile ``csrc/torch_ops.cpp`` (the entry points registered as ``torch.ops.tokquay_amd.*``)
    against torch's headers and libraries; it links LIB_PATH. Returns its path."""
    import torch
    from torch.utils import cpp_extension

    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler (g++) found")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    torch_lib = cpp_extension.library_paths()[0]
    tmp = TORCH_OPS_PATH + ".tmp"
    # torch's HIP stream header includes the HIP runtime's, which needs the platform named when the
    # host compiler is not hipcc.
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", *[f"-I{p}" for p in cpp_extension.include_paths()], f"-I{ROCM_INCLUDE}",
           f"-I{INCLUDE_DIR}", "-o", tmp, TORCH_OPS_SRC, f"-L{PKG_DIR}", "-l:" + LIB_NAME, f"-L{torch_lib}",
           "-lc10", "-lc10_hip", "-ltorch_cpu", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]  # fmt: skip
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{cxx} failed ({proc.returncode}):\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, TORCH_OPS_PATH)
    return TORCH_OPS_PATH


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv[1:]))
