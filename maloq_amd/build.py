"""Builds libmaloq_hip.so (all HIP kernels + the C ABI) in-tree for gfx950,
then the PyTorch operator layer _maloq_torch.so (a C++ extension over it).

Usage: python -m maloq_amd.build   (or __graft_entry__.build()).
Each .hip file is compiled to an object in parallel, then linked; the results
are maloq_amd/libmaloq_hip.so and maloq_amd/_maloq_torch.so next to this file.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libmaloq_hip.so")
BUILD_DIR = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# The PyTorch operator layer (torch_ops.cpp): a C++ extension built with g++
# against torch's headers, linking libmaloq_hip.so.
TORCH_SRC = os.path.join(CSRC, "torch_ops.cpp")
TORCH_EXT = os.path.join(HERE, "_maloq_torch.so")
CXX = os.environ.get("CXX", "g++")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


_INCLUDE = re.compile(r'^\s*#\s*include\s+"([^"]+)"', re.M)


def _deps(path: str, seen: set) -> set:
    """The file and every project header it includes, transitively."""
    path = os.path.normpath(path)
    if path in seen or not os.path.exists(path):
        return seen
    seen.add(path)
    with open(path, encoding="utf-8", errors="replace") as f:
        for inc in _INCLUDE.findall(f.read()):
            _deps(os.path.join(os.path.dirname(path), inc), seen)
    return seen


def _deps_mtime(src: str) -> float:
    """Newest mtime among the source and the headers it includes."""
    return max(os.path.getmtime(p) for p in _deps(src, set()))


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    if incremental and os.path.exists(obj) and os.path.getmtime(obj) >= _deps_mtime(src):
        return obj
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True, incremental: bool = False) -> str:
    """Compile every HIP source (``incremental`` reuses objects newer than their
    inputs; the default always recompiles)."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    # the kernel-heavy units (template instantiations of the message block)
    # start first, then the rest, largest first
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")),
                  key=lambda f: ("message_l" not in os.path.basename(f), -os.path.getsize(f), f))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, incremental), srcs))
    tmp = OUT + ".tmp"
    # -Bsymbolic: the library's calls to its own functions (the per-shape launch
    # templates, kernel stubs) bind inside it.  Without it they go through the
    # PLT, and a second build loaded into the same process (a copy with other
    # tile sizes, another version) would run the first build's definitions with
    # its own sizes.
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-Bsymbolic", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources", flush=True)
    return OUT


def build_torch_ext(verbose: bool = True, incremental: bool = False) -> str:
    """Compile the operator layer into maloq_amd/_maloq_torch.so (after the
    HIP library, which it links)."""
    if incremental and os.path.exists(TORCH_EXT) and os.path.getmtime(TORCH_EXT) >= _deps_mtime(TORCH_SRC):
        return TORCH_EXT
    import torch

    tdir = os.path.dirname(torch.__file__)
    inc = [os.path.join(tdir, "include"), os.path.join(tdir, "include", "torch", "csrc", "api", "include")]
    libdir = os.path.join(tdir, "lib")
    tmp = TORCH_EXT + ".tmp"
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
           "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-I{p}" for p in inc], "-I/opt/rocm/include", TORCH_SRC, "-o", tmp,
           f"-L{HERE}", "-lmaloq_hip", f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch extension build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, TORCH_EXT)
    if verbose:
        print(f"built {TORCH_EXT}", flush=True)
    return TORCH_EXT


if __name__ == "__main__":
    build(incremental="--incremental" in sys.argv)
    build_torch_ext(incremental="--incremental" in sys.argv)
    sys.exit(0)
