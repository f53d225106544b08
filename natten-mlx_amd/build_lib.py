"""Build libnatten_amd.so (the C-ABI HIP library) in-tree for gfx950.

Usage: python natten-mlx_amd/build_lib.py [--jobs N] [--verbose]

Each csrc/*.hip file is compiled separately (in parallel) with hipcc and the
objects are linked into natten-mlx_amd/natten_amd/libnatten_amd.so, which the
Python package loads with ctypes; csrc/na_torch.cpp (the fused op's torch
custom operator over that library) is compiled with the host compiler into
natten_amd/libnatten_amd_torch.so.  The build always recompiles, so it is a
real "does it build" check.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(HERE, "natten_amd", "libnatten_amd.so")
OP_PATH = os.path.join(HERE, "natten_amd", "libnatten_amd_torch.so")

ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # packed fp32 VALU ops are kept off for every kernel of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    "-I", INCLUDE,
    "-I", CSRC,
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP toolchain is required")
    return path


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


# Per-file extra flags.  The matrix-core kernels keep MFMA accumulators in
# ordinary VGPRs (gfx950 allows it), which removes the AGPR<->VGPR copies
# their softmax arithmetic would otherwise need.
EXTRA_FLAGS = {
    "na_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "na_lean.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "na_dense.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(os.path.basename(src), []), "-c", src,
           "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 1, 8)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libnatten_amd.so",
           *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    build_torch_op(verbose)
    return LIB_PATH


def build_torch_op(verbose: bool = False) -> str:
    """libnatten_amd_torch.so: the fused op as a torch custom operator with
    its autograd node in C++ (csrc/na_torch.cpp), compiled with the host
    compiler against torch's headers and linked to libnatten_amd.so."""
    import torch
    from torch.utils import cpp_extension

    cxx = shutil.which("g++") or "c++"
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    incs = [f"-I{p}" for p in cpp_extension.include_paths()]
    libdirs = cpp_extension.library_paths()
    tmp = OP_PATH + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-I", INCLUDE, *incs, os.path.join(CSRC, "na_torch.cpp"), "-o", tmp,
           *[f"-L{d}" for d in libdirs], "-ltorch", "-ltorch_cpu", "-lc10",
           f"-L{os.path.dirname(LIB_PATH)}", "-lnatten_amd",
           "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{d}" for d in libdirs]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch op build failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OP_PATH)
    return OP_PATH


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(args.jobs, args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
