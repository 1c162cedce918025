"""Build recipe for libmoe_mi355.so (hipcc, gfx950 only) and its torch binding.

Each ``csrc/*.hip`` file is compiled to an object in ``csrc/_build/`` (in
parallel) and the objects are linked into ``moe_mi355/libmoe_mi355.so``.  The
library has no torch dependency: it exports the plain C ABI declared in
``include/moe_mi355.h`` and is loaded with ctypes.

``csrc/torch_router.cpp`` (host code only) is then compiled against torch's
headers into the Python extension ``moe_mi355/_moe_torch.so``: the router's
autograd Function in C++, calling the same C ABI (it links libmoe_mi355.so
from its own directory).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(ROOT, "csrc")
BUILD = os.path.join(CSRC, "_build")
LIB = os.path.join(PKG_DIR, "libmoe_mi355.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Keep the compiler from forming packed fp32 ops (v_pk_*_f32).
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmoe_mi355.so)")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(hipcc: str, src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


TORCH_EXT = os.path.join(PKG_DIR, "_moe_torch.so")


def build_torch_binding(hipcc: str) -> str:
    """Compile csrc/torch_router.cpp into moe_mi355/_moe_torch.so (needs libmoe_mi355.so built first)."""
    import sysconfig

    import torch
    import torch.utils.cpp_extension as ce

    src = os.path.join(CSRC, "torch_router.cpp")
    obj = os.path.join(BUILD, "torch_router.o")
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    incs = ["-I/opt/rocm/include"] + [f"-I{p}" for p in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}"]
    cmd = [hipcc, "-x", "c++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           "-DTORCH_API_INCLUDE_EXTENSION_H", "-DTORCH_EXTENSION_NAME=_moe_torch", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *incs, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed for {src}:\n{res.stdout}\n{res.stderr}")
    tmp = TORCH_EXT + ".tmp"
    libs = [f"-L{p}" for p in ce.library_paths()] + ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
                                                      "-ltorch_python"]
    cmd = [hipcc, "-shared", "-fPIC", obj, f"-L{PKG_DIR}", "-l:libmoe_mi355.so", "-Wl,-rpath,$ORIGIN", *libs,
           "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed for {TORCH_EXT}:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, TORCH_EXT)
    return TORCH_EXT


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip file and link libmoe_mi355.so, then the torch binding; returns the library's
    path."""
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s), srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    build_torch_binding(hipcc)
    if verbose:
        print(f"built {TORCH_EXT}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
