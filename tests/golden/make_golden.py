"""Writes tests/golden/cfg1_golden.npz: the config-1 workload's expected
attention output and lse from the CPU oracle, plus a SHA-256 of the generated
inputs so a test can confirm it regenerated the same bits.

The reference commits no golden vectors for this path (its only data-driven
driver reads an absent dataset file), so these fixtures pin the oracle and the
HIP path against regressions; the oracle itself is pinned by
tests/test_oracle.py.  Run from the repository root:

    python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flashinfer-repo_amd")]

import torch  # noqa: E402

import oracle  # noqa: E402
from dsa_amd import workloads  # noqa: E402


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def input_digest(d) -> str:
    h = hashlib.sha256()
    for k in ("q_nope", "q_pe", "ckv_cache", "kpe_cache"):
        h.update(bits(d[k]).tobytes())
    h.update(d["sparse_indices"].numpy().astype(np.int32).tobytes())
    return h.hexdigest()


def main():
    d = workloads.cfg1()
    out, lse = oracle.attention(bits(d["q_nope"]), bits(d["q_pe"]), bits(d["ckv_cache"]),
                                bits(d["kpe_cache"]), d["sparse_indices"].numpy(), d["sm_scale"])
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg1_golden.npz")
    np.savez_compressed(path, out_bits=out, lse=lse, sparse_indices=d["sparse_indices"].numpy(),
                        input_sha256=np.array(input_digest(d)), sm_scale=np.float32(d["sm_scale"]))
    print(path, input_digest(d))


if __name__ == "__main__":
    main()
