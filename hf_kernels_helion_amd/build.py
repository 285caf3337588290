"""Build libfp8_blockwise.so (gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: python -m hf_kernels_helion_amd.build   (or build() from Python)
The library has no torch dependency; the Python package loads it with ctypes.
Beside it: libfp8_torch_ops.so (the torch custom ops) and _fp8_fast.so (direct
Python bindings of the hot ops for eager calls).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "_lib"
LIB_NAME = "libfp8_blockwise.so"
TORCH_LIB_NAME = "libfp8_torch_ops.so"
FAST_MODULE_NAME = "_fp8_fast.so"
SOURCES = ["capi.cpp", "act_quant.hip", "block_gemm.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def compile_flags() -> list:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Keep hipcc from forming packed fp32 (v_pk_*_f32) instructions.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
    ]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build_torch_ops(verbose: bool = False) -> Path:
    """Compile the torch custom-op library (host C++ only) against torch's
    headers; it links libfp8_blockwise.so from the same directory."""
    import torch
    from torch.utils import cpp_extension as ce
    out = LIB_DIR / TORCH_LIB_NAME
    tmp = LIB_DIR / (TORCH_LIB_NAME + ".tmp")
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=fp8_torch_ops", "-Wno-deprecated-declarations"]
    for inc in ce.include_paths(device_type="cuda"):
        cmd += ["-isystem", inc]
    cmd += [str(CSRC / "torch_ops.cpp"), "-o", str(tmp),
            f"-L{LIB_DIR}", "-lfp8_blockwise", f"-L{torch_lib}", "-lc10", "-lc10_hip",
            "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-Wl,-rpath,$ORIGIN",
            f"-Wl,-rpath,{torch_lib}"]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build_fast_module(verbose: bool = False) -> Path:
    """Compile the direct Python bindings of the hot ops (torch_fast.cpp) into
    the extension module LIB_DIR/_fp8_fast.so; it links the op library."""
    import sysconfig
    import torch
    from torch.utils import cpp_extension as ce
    out = LIB_DIR / FAST_MODULE_NAME
    tmp = LIB_DIR / (FAST_MODULE_NAME + ".tmp")
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-DTORCH_EXTENSION_NAME=_fp8_fast", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-Wno-deprecated-declarations", "-fvisibility=hidden"]
    for inc in ce.include_paths(device_type="cuda") + [sysconfig.get_paths()["include"]]:
        cmd += ["-isystem", inc]
    cmd += [str(CSRC / "torch_fast.cpp"), "-o", str(tmp),
            f"-L{LIB_DIR}", "-lfp8_torch_ops", f"-L{torch_lib}", "-lc10", "-ltorch",
            "-ltorch_cpu", "-ltorch_python", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    """Compile the HIP kernels into LIB_DIR/LIB_NAME and the torch op library
    beside it; returns the kernel library path."""
    LIB_DIR.mkdir(exist_ok=True)
    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), *compile_flags(), "-shared", "-o", str(tmp)]
    cmd += [str(CSRC / s) for s in SOURCES]
    _run(cmd, verbose)
    os.replace(tmp, out)
    build_torch_ops(verbose)
    build_fast_module(verbose)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
