"""Builds the gfx950 shared library ``libresihp_moe.so`` from ``csrc/`` with hipcc.

    python resihp-megatron_amd/build.py        # or call build() from Python

Every HIP source is compiled for gfx950 only, with packed-FP32 instructions
disabled, into ``_build/``; the objects are linked into
``libresihp_moe.so`` next to this file.  The library exports the C ABI
declared in ``include/resihp_moe.h``.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "_build"
LIB = PKG / "libresihp_moe.so"
INCLUDE = PKG.parent / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{INCLUDE}"]


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = OUT / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> pathlib.Path:
    """Compiles every source in csrc/ and links libresihp_moe.so; returns its path."""
    OUT.mkdir(exist_ok=True)
    sources = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.cpp")])
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
