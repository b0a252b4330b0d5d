"""Builds libmgopt.so (the HIP kernels and C ABI) for gfx950, in-tree.

Run as a script or call build().  The library lands in _build/ next to this
file; the Python host layer loads it from there and nowhere else.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "csrc" / "mgopt.hip"
INCLUDE = HERE.parent / "include"
OUT_DIR = HERE / "_build"
LIB = OUT_DIR / "libmgopt.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # every fused multiply-add in the kernels is written out explicitly
    "-ffp-contract=off",
    # no packed-fp32 instructions (v_pk_*_f32) anywhere in the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libmgopt.so)")


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", str(SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    noise = [ln for ln in proc.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if verbose and noise:
        print("\n".join(noise), file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


HOST_SRC = HERE / "csrc" / "host_ptrs.cpp"
HOST_DIR = OUT_DIR / "host"


def build_host(verbose: bool = False) -> Path:
    """Builds the host-side helper (a torch C++ extension) into _build/host/."""
    from torch.utils.cpp_extension import load

    if HOST_DIR.exists():
        shutil.rmtree(HOST_DIR)
    HOST_DIR.mkdir(parents=True)
    load(name="mgopt_host", sources=[str(HOST_SRC)], build_directory=str(HOST_DIR), extra_cflags=["-O2"],
         verbose=verbose)
    return HOST_DIR / "mgopt_host.so"


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_host(verbose=False))
