"""Build the gfx950 HIP library ``libmoe_hip.so`` in-tree with hipcc.

The library is a plain C-ABI shared object (see include/moe_hip.h); it is
loaded with ctypes, so it is built directly with hipcc rather than as a torch
C++ extension and carries no torch headers or C++ ABI.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(REPO_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libmoe_hip.so")
# Python binding of the two drop-in entry points (csrc/torch_bind.cpp):
# host C++ against torch's C++ API, no HIP; it allocates the outputs in C++
# and calls the library through addresses taken from ctypes.
FAST_NAME = "_moe_torch"
FAST_PATH = os.path.join(PKG_DIR, FAST_NAME + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))

SOURCES = ["router.hip", "gemm.hip", "router_gemm.hip", "moe.hip", "capi.cpp"]
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-I", os.path.join(REPO_DIR, "include"),
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libmoe_hip.so")
    return path


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, *lang, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(extra_flags: list[str] | None = None, verbose: bool = False) -> str:
    """Compile every source for gfx950 and link ``libmoe_hip.so``; returns its path."""
    extra = list(extra_flags or [])
    os.makedirs(BUILD_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as ex:
        fast = ex.submit(build_fast)
        objs = list(ex.map(lambda s: _compile(s, extra), SOURCES))
        fast.result()
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} and {FAST_PATH}")
    return LIB_PATH


def build_fast() -> str:
    """Compile the torch binding csrc/torch_bind.cpp in-tree with the host C++ compiler."""
    import torch
    from torch.utils import cpp_extension as ce

    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no C++ compiler (g++) found for the torch binding")
    abi = int(bool(getattr(torch._C, "_GLIBCXX_USE_CXX11_ABI", True)))
    inc = [f"-I{p}" for p in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}", "-I/opt/rocm/include"]
    libs = [f"-L{p}" for p in ce.library_paths()] + [f"-Wl,-rpath,{p}" for p in ce.library_paths()]
    tmp = FAST_PATH + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-w", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-DTORCH_EXTENSION_NAME={FAST_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H", *inc,
           os.path.join(CSRC, "torch_bind.cpp"), "-o", tmp, *libs, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_python"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the torch binding failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, FAST_PATH)
    return FAST_PATH


if __name__ == "__main__":
    build(verbose=True)
