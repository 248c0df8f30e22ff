"""Build libluxgpu_backend_hip.so in-tree with hipcc for gfx950.

The plugin is compiled from mlx_amd/csrc/*.hip (hipcc, gfx950) and the
host-only mlx_amd/csrc/*.cpp (g++) into mlx_amd/lib/.  Every
source is compiled each time build() runs (the driver's "does it build"
check); objects land in mlx_amd/_build/ and are linked into one shared
library whose only exported symbols are the two plugin entry points;
csrc/core/lux_quant_core.cpp builds the separate core-side library.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
PLUGIN = os.path.join(LIBDIR, "libluxgpu_backend_hip.so")
CORE = os.path.join(LIBDIR, "libluxgpu_quant_core.so")
CORE_SRC = os.path.join(CSRC, "core", "lux_quant_core.cpp")
# bench.py's ceiling leg (empty kernel, plain read): its own library, not the plugin
CEILING = os.path.join(LIBDIR, "libluxgpu_ceiling.so")
CEILING_SRC = os.path.join(CSRC, "probe", "ceiling.hip")
ARCH = os.environ.get("LUX_HIP_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    # packed fp32 VALU ops are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # device code objects stored compressed in the library (the HIP runtime
    # expands them when it loads the module): about a quarter of the size
    "--offload-compress",
]


CXX = os.environ.get("CXX", "g++")
CXXFLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra"]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    if src.endswith(".cpp"):
        cmd = [CXX, *CXXFLAGS, "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def sources() -> list:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = PLUGIN + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, PLUGIN)
    build_core()
    build_ceiling()
    if verbose:
        print(f"built {PLUGIN}, {CORE} and {CEILING}", file=sys.stderr)
    return PLUGIN


def build_core() -> str:
    """The core-side selection library: host C++ only, linked with libdl."""
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = CORE + ".tmp"
    cmd = [CXX, *CXXFLAGS, "-shared", CORE_SRC, "-ldl", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"core library build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, CORE)
    return CORE


def build_ceiling() -> str:
    """bench.py's measurement kernels (csrc/probe/ceiling.hip)."""
    os.makedirs(LIBDIR, exist_ok=True)
    tmp = CEILING + ".tmp"
    cmd = [HIPCC, *CFLAGS, "-shared", CEILING_SRC, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ceiling library build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, CEILING)
    return CEILING


if __name__ == "__main__":
    build(verbose=True)
