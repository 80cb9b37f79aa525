"""Shared test setup.

* ``gpu`` marks tests that need an MI355X; everything else runs on the CPU.
* The repository root (for ``oracle``) and ``flashinfer-repo_amd`` (for the
  ``dsa_amd`` package) are put on ``sys.path``.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "flashinfer-repo_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

# Tolerances of the reference's checker (docs/CORRECTNESS.md:23-36): an
# element fails only if it exceeds BOTH the absolute and the relative bound.
OUT_ATOL = OUT_RTOL = 1e-2   # bf16 output
LSE_ATOL = LSE_RTOL = 1e-3   # fp32 base-2 lse


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (run with -m gpu)")


def mismatches(actual, expected, atol, rtol):
    """Count elements with |a-e| > atol AND |a-e| > rtol*|e| (inf/-inf must match)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    both_inf = np.isinf(a) & np.isinf(e) & (np.sign(a) == np.sign(e))
    with np.errstate(invalid="ignore"):  # inf - inf where both are -inf (empty rows' lse)
        diff = np.abs(a - e)
    bad = (diff > atol) & (diff > rtol * np.abs(e))
    bad |= np.isnan(a) != np.isnan(e)
    bad &= ~both_inf
    bad |= np.isinf(a) != np.isinf(e)
    bad |= np.isinf(a) & np.isinf(e) & (np.sign(a) != np.sign(e))  # +inf against -inf
    return int(bad.sum())


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    return oracle


LDS_POISON_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liblds_poison.so")
# NaN as fp32 and as each of its bf16 halves; a negative int32
LDS_POISON_PATTERN = 0xFFC0FFC0
_poison = None


def fill_lds_with_nan(device):
    """Leaves a NaN bit pattern in the whole LDS of every CU: 4096 workgroups
    of the test-support kernel in tests/lds_poison.hip (built by
    ``__graft_entry__.build()``), each taking all 160 KB of a CU's LDS and
    writing the pattern over it.  LDS is not cleared between workgroups, so a
    kernel launched next on the same stream that reads an LDS location before
    writing it computes with NaN (or a negative slot id), which the parity
    checks see."""
    import ctypes

    import torch
    global _poison
    if _poison is None:
        if not os.path.exists(LDS_POISON_LIB):
            raise RuntimeError(f"{LDS_POISON_LIB} is missing: run __graft_entry__.build() first")
        lib = ctypes.CDLL(LDS_POISON_LIB)
        lib.lds_poison_fill.argtypes = [ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p]
        lib.lds_poison_fill.restype = ctypes.c_int
        _poison = lib
    dev = torch.device(device)
    stream = torch._C._cuda_getCurrentRawStream(dev.index if dev.index is not None else 0)
    rc = _poison.lds_poison_fill(LDS_POISON_PATTERN, 4096, stream)
    if rc != 0:
        raise RuntimeError(f"lds_poison_fill failed with HIP status {rc}")
