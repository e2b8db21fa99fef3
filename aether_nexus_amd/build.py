"""Build the gfx950 Weaver library in-tree (``aether_nexus_amd/libaether_weaver.so``).

The reference compiles its Metal shaders in build.rs (xcrun metal -> metallib,
nexus-core/build.rs:14-82); here hipcc compiles the HIP sources for gfx950
into one shared library that exports the C ABI of include/aether_weaver.h.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SOURCES = [PKG / "csrc" / "weaver_engine.hip", PKG / "csrc" / "fabric.hip", PKG / "csrc" / "ops.hip"]
DEPS = [PKG / "csrc" / "weaver_kernels.hpp", PKG / "csrc" / "ops_kernels.hpp", PKG / "csrc" / "engine_internal.hpp",
        ROOT / "include" / "aether_weaver.h", ROOT / "include" / "aether_fabric.h", ROOT / "include" / "aether_ops.h"]
OUT = PKG / "libaether_weaver.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    # gfx950's packed fp32 instructions stay off: hipcc is not allowed to form them.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm required to build the gfx950 library)")
    return path


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into OUT (always recompiles)."""
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(ROOT / "include"), "-o", str(tmp), *map(str, SOURCES)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature and says so; drop that noise.
    noise = "packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
