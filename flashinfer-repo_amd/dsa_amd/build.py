"""Builds libdsa_amd.so in-tree with hipcc for gfx950.

The library is a plain C-ABI shared object (see include/dsa_abi.h); it is
compiled with hipcc directly, not through a framework extension builder, so
that nothing framework-specific crosses its boundary.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(os.path.dirname(PKG_DIR), "csrc")
LIB_PATH = os.path.join(PKG_DIR, "libdsa_amd.so")

SOURCES = ["dsa_abi.cpp", "dsa_attention.hip", "dsa_indexer.hip", "dsa_noalloc.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # fused multiply-adds stay on, but `#pragma clang fp contract(off)` is
    # honoured (the indexer score defines its rounding order)
    "-ffp-contract=fast-honor-pragmas",
    # Packed-fp32 VALU forms are kept out of every code object.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def build(verbose: bool = False) -> str:
    """Compile every HIP source into ``libdsa_amd.so``; returns its path."""
    srcs = [os.path.join(CSRC_DIR, s) for s in SOURCES]
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", tmp, *srcs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    if verbose and out.strip():
        print(out, flush=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB_PATH)
