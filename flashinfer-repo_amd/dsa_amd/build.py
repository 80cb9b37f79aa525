"""Builds libdsa_amd.so in-tree with hipcc for gfx950.

The library is a plain C-ABI shared object (see include/dsa_abi.h); it is
compiled with hipcc directly, not through a framework extension builder, so
that nothing framework-specific crosses its boundary.  Every source is
compiled to an object of its own (in parallel) under ``_build/``, then
linked.

``build(sanitize=True)`` also links ``libdsa_amd_san.so``: the same kernel
objects with the host-side C-ABI sources (argument validation, launch
configuration, the scratch-array setup) compiled with AddressSanitizer and
UndefinedBehaviorSanitizer on the host pass only.  ``tests/test_abi_sanitized.py``
runs the CPU ABI tests against it.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC_DIR = os.path.join(os.path.dirname(PKG_DIR), "csrc")
BUILD_DIR = os.path.join(os.path.dirname(PKG_DIR), "_build")
LIB_PATH = os.path.join(PKG_DIR, "libdsa_amd.so")
SAN_LIB_PATH = os.path.join(PKG_DIR, "libdsa_amd_san.so")

SOURCES = ["dsa_abi.cpp", "dsa_attention.hip", "dsa_indexer.hip", "dsa_noalloc.hip"]
# host-side C-ABI code: validation, launch configuration, scratch-array setup
HOST_ABI_SOURCES = ["dsa_abi.cpp", "dsa_noalloc.hip"]

COMMON_FLAGS = [
    "--offload-arch=gfx950",
    "-std=c++17",
    "-fPIC",
    # fused multiply-adds stay on, but `#pragma clang fp contract(off)` is
    # honoured (the indexer score defines its rounding order)
    "-ffp-contract=fast-honor-pragmas",
    # Packed-fp32 VALU forms are kept out of every code object.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
OPT_FLAGS = ["-O3"]
# AddressSanitizer + UndefinedBehaviorSanitizer on the host pass only (the GPU
# code objects are the product's own).
SAN_FLAGS = ["-O1", "-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=all"]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


def _filter(out: str) -> str:
    return "\n".join(l for l in out.splitlines()
                     if "packed-fp32-ops" not in l and "hip-link" not in l)


def _run_all(cmds, verbose: bool) -> None:
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                            text=True)))
    failed = []
    for cmd, pr in procs:
        out = _filter(pr.communicate()[0])
        if pr.returncode != 0:
            failed.append(f"{' '.join(cmd)}\n{out}")
        elif verbose and out.strip():
            print(out, flush=True)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n\n".join(failed))


def _obj(src: str, tag: str) -> str:
    return os.path.join(BUILD_DIR, f"{os.path.splitext(src)[0]}{tag}.o")


def build(verbose: bool = False, sanitize: bool = False) -> str:
    """Compile every HIP source and link ``libdsa_amd.so`` (and, with
    ``sanitize``, ``libdsa_amd_san.so``); returns the product library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    cc = hipcc()
    compiles = [[cc, *COMMON_FLAGS, *OPT_FLAGS, "-c", "-o", _obj(s, ""), os.path.join(CSRC_DIR, s)]
                for s in SOURCES]
    if sanitize:
        compiles += [[cc, *COMMON_FLAGS, *SAN_FLAGS, "-c", "-o", _obj(s, ".san"),
                      os.path.join(CSRC_DIR, s)] for s in HOST_ABI_SOURCES]
    _run_all(compiles, verbose)
    links = []
    tmp = LIB_PATH + ".tmp"
    links.append([cc, *COMMON_FLAGS, "-shared", "-o", tmp, *[_obj(s, "") for s in SOURCES]])
    if sanitize:
        objs = [_obj(s, ".san" if s in HOST_ABI_SOURCES else "") for s in SOURCES]
        links.append([cc, *COMMON_FLAGS, "-shared", "-Xarch_host", "-fsanitize=address",
                      "-Xarch_host", "-fsanitize=undefined", "-shared-libsan", "-o",
                      SAN_LIB_PATH + ".tmp", *objs])
    _run_all(links, verbose)
    os.replace(tmp, LIB_PATH)
    if sanitize:
        os.replace(SAN_LIB_PATH + ".tmp", SAN_LIB_PATH)
    return LIB_PATH


def build_test_support(src: str, lib: str, verbose: bool = False) -> str:
    """Compile one self-contained HIP source of the tests (not part of the
    product library) into its own shared object ``lib``."""
    tmp = lib + ".tmp"
    _run_all([[hipcc(), *COMMON_FLAGS, *OPT_FLAGS, "-shared", "-o", tmp, src]], verbose)
    os.replace(tmp, lib)
    return lib


def sanitizer_runtime() -> str:
    """The AddressSanitizer runtime of ROCm's clang (to LD_PRELOAD into a
    process that loads libdsa_amd_san.so)."""
    out = subprocess.run([hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"],
                         stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True).stdout.strip()
    if not os.path.isabs(out) or not os.path.exists(out):
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        base = os.path.join(rocm, "llvm", "lib", "clang")
        for ver in sorted(os.listdir(base)) if os.path.isdir(base) else []:
            cand = os.path.join(base, ver, "lib", "linux", "libclang_rt.asan-x86_64.so")
            if os.path.exists(cand):
                return cand
    return out


if __name__ == "__main__":
    build(verbose="-v" in sys.argv, sanitize="--sanitize" in sys.argv)
    print(LIB_PATH)
