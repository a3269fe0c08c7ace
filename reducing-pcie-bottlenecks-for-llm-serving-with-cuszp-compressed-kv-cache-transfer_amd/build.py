"""Builds libkvszp.so (HIP kernels + C ABI) for gfx950, in place.

    python build.py            # compile csrc/*.hip + csrc/*.cpp -> libkvszp.so,
                               # csrc/kvszp_torch_args.cpp -> kvszp_torch_args.so

Flags: no fast-math and no floating-point contraction (the quantizer and the
decoder must round every fp32 operation exactly once), packed-fp32 code
generation disabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
LIB_NAME = "libkvszp.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = os.environ.get("KVSZP_ARCH", "gfx950")

SOURCES = ["kvszp_kernels.hip", "kvszp_capi.cpp"]
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc",
                 shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


ARGS_NAME = "kvszp_torch_args"
ARGS_PATH = os.path.join(HERE, ARGS_NAME + ".so")


def build_args_helper(verbose: bool = False) -> str:
    """Compiles csrc/kvszp_torch_args.cpp, the drop-in module's argument
    marshalling helper (host C++ against torch's headers, no device code),
    to kvszp_torch_args.so next to this file; returns its path."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    obj = os.path.join(build_dir, ARGS_NAME + ".o")
    flags = [f"-DTORCH_EXTENSION_NAME={ARGS_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
             f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
             "-O2", "-fPIC", "-std=c++17"]
    for inc in cpp_extension.include_paths():
        flags += ["-isystem", inc]
    flags += ["-isystem", sysconfig.get_paths()["include"]]
    cmd = ["g++", *flags, "-c", os.path.join(CSRC, ARGS_NAME + ".cpp"), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp = ARGS_PATH + ".tmp"
    cmd = ["g++", "-shared", obj, "-o", tmp]
    for lib_dir in cpp_extension.library_paths():
        cmd += ["-L", lib_dir]
    cmd += ["-lc10", "-ltorch_cpu", "-ltorch", "-ltorch_python"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, ARGS_PATH)
    return ARGS_PATH


def build(verbose: bool = False) -> str:
    """Compile every source and link the shared library; returns its path."""
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    objects = []
    for src in SOURCES:
        obj = os.path.join(build_dir, src + ".o")
        cmd = [hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c",
               os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objects.append(obj)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp,
           *objects]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB_PATH)
    build_args_helper(verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
