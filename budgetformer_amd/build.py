"""Build recipe for the HIP library behind the C ABI (include/budgetformer_hip.h).

Compiles every ``csrc/*.hip`` for gfx950 with hipcc and links
``budgetformer_amd/_lib/libbudgetformer_hip.so`` in-tree (the .so travels
with the source tree; nothing is installed). ``python -m budgetformer_amd.build``
runs it.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT_DIR = os.path.join(PKG, "_lib")
LIB_NAME = "libbudgetformer_hip.so"
ARCH = os.environ.get("BF_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed-fp32 instructions are kept out of the generated code on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]
# Extra compile definitions for tuning sweeps (e.g. "-DBF_UNROLL_FWD_F32=2"); empty by default.
HIPCC_FLAGS += os.environ.get("BF_HIPCC_EXTRA", "").split()


OPS_NAME = "libbf_torch_ops.so"


def lib_path() -> str:
    return os.path.join(OUT_DIR, LIB_NAME)


def ops_path() -> str:
    return os.path.join(OUT_DIR, OPS_NAME)


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP library)")


def _compile(hipcc: str, src: str, obj: str) -> None:
    cmd = [hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # the host pass does not know the packed-fp32 feature; that warning is expected
    noise = "is not a recognized feature for this target"
    out = "\n".join(l for l in res.stdout.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = True) -> str:
    """Compile all HIP sources and link the shared library; returns its path."""
    hipcc = _hipcc()
    os.makedirs(OUT_DIR, exist_ok=True)
    obj_dir = os.path.join(OUT_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = [os.path.join(obj_dir, s[:-4] + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(len(srcs), 4)) as ex:
        futs = [ex.submit(_compile, hipcc, os.path.join(CSRC, s), o) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = lib_path() + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}")
    os.replace(tmp, lib_path())
    if verbose:
        print(f"[budgetformer_amd] built {lib_path()}")
    build_torch_ops(verbose)
    return lib_path()


def build_torch_ops(verbose: bool = True) -> str:
    """The TORCH_LIBRARY(bf, ...) operators (csrc/torch_ops.cpp): host C++ against PyTorch's headers,
    linked to the HIP library beside it (rpath $ORIGIN); loaded with torch.ops.load_library."""
    import torch
    from torch.utils import cpp_extension

    src = os.path.join(CSRC, "torch_ops.cpp")
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    incs = [f"-I{p}" for p in cpp_extension.include_paths()] + ["-I/opt/rocm/include", f"-I{os.path.join(ROOT, 'include')}"]
    libdir = cpp_extension.library_paths()[0]
    tmp = ops_path() + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           # the platform macro HIP's runtime headers (included by PyTorch's c10/hip) require
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", *incs, src, "-o", tmp,
           f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           f"-L{OUT_DIR}", "-lbudgetformer_hip", "-L/opt/rocm/lib", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch_ops build failed:\n{res.stdout}")
    if res.stdout.strip():
        print(res.stdout, file=sys.stderr)
    os.replace(tmp, ops_path())
    if verbose:
        print(f"[budgetformer_amd] built {ops_path()}")
    return ops_path()


if __name__ == "__main__":
    build()
