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


def fill_lds_with_nan(device):
    """Leaves NaN bit patterns in the LDS of every CU: a bf16 GEMM of NaN
    operands (4096^3, more than one workgroup per CU) stages its tiles there,
    and LDS is not cleared between workgroups.  A kernel launched next on the
    same stream that reads an LDS location before writing it then computes
    with NaN, which the parity checks see."""
    import torch
    a = torch.full((4096, 4096), float("nan"), dtype=torch.bfloat16, device=device)
    return a @ a
