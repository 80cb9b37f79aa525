"""Replay of recorded DSA workloads stored as safetensors files.

The reference's correctness driver (test_splitk_correctness.py:6-18) takes
the ``sparse_indices`` of one recorded workload from a safetensors file of
the contest dataset (workloads/dsa_paged/<definition>/<definition>_<uuid>
.safetensors), draws the queries and the paged cache at random with the
definition's shapes (num_tokens = 1, 8462 pages of 64 rows, H = 16), and
compares ``kernel`` with ``kernel_splitk`` for several split counts.  The
dataset itself is not part of this repository; these helpers do the same for
any such file (or any file holding an int32 ``[T, topk]`` index tensor), with
the inputs drawn on the CPU from a seed so that a CPU checker sees the same
bits.  Files are read with ``safetensors`` (no code is executed from them).
"""
from __future__ import annotations

import math
from typing import Dict, Optional

import torch

from . import workloads


def load_sparse_indices(path: str, key: str = "sparse_indices") -> torch.Tensor:
    """The ``[T, topk]`` slot-id tensor of a recorded workload, as int32.

    Raises ``KeyError`` if the file has no tensor ``key`` and ``ValueError`` if
    it is not a 2-D integer tensor."""
    from safetensors.torch import load_file
    tensors = load_file(path, device="cpu")
    if key not in tensors:
        raise KeyError(f"{path}: no tensor '{key}' (has: {sorted(tensors)})")
    idx = tensors[key]
    if idx.dim() != 2 or idx.dtype.is_floating_point or idx.dtype == torch.bool:
        raise ValueError(f"{path}: '{key}' must be a 2-D integer tensor, got {idx.dtype} "
                         f"{tuple(idx.shape)}")
    return idx.to(torch.int32).contiguous()


def workload_inputs(sparse_indices: torch.Tensor, num_pages: int, page_size: int = 64,
                    num_heads: int = 16, sm_scale: Optional[float] = None,
                    seed: int = 0) -> Dict[str, object]:
    """Inputs around recorded indices, shaped as the reference driver draws
    them: q_nope/q_pe ~ N(0, 1), ckv/kpe ~ N(0, 1), bf16, paged
    ``[num_pages, page_size, D]``.  Raises ``ValueError`` if an index is at or
    beyond ``num_pages * page_size`` (the reference's run() would fail on it)."""
    T = sparse_indices.shape[0]
    hi = int(sparse_indices.max()) if sparse_indices.numel() else -1
    if hi >= num_pages * page_size:
        raise ValueError(f"slot id {hi} is beyond the cache ({num_pages} pages of {page_size})")
    d = workloads.attention_inputs(T, num_heads, sparse_indices.shape[1], num_pages, page_size,
                                   seed, cache_var=1.0)
    d.pop("gen")
    d.update(sparse_indices=sparse_indices.to(torch.int32).contiguous(),
             sm_scale=float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(192.0))
    return d


def replay(path: str, num_pages: int, page_size: int = 64, num_heads: int = 16,
           sm_scale: Optional[float] = None, seed: int = 0, device="cuda",
           split_ks=(4, 8, 16)) -> Dict[str, float]:
    """Runs ``kernel`` and ``kernel_splitk`` (each of ``split_ks``) on one
    recorded workload, as the reference driver does, and returns the largest
    |difference| of the output and the lse for each split count."""
    from .kernel import kernel, kernel_splitk
    d = workload_inputs(load_sparse_indices(path), num_pages, page_size, num_heads, sm_scale,
                        seed)
    g = workloads.to_device(d, device)
    args = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], g["sparse_indices"],
            d["sm_scale"])
    out, lse = kernel(*args)
    errs = {}
    for s in split_ks:
        o, l = kernel_splitk(*args, SPLIT_K=s)
        errs[f"split{s}_out"] = float((out.float() - o.float()).abs().max())
        fin = torch.isfinite(lse)
        errs[f"split{s}_lse"] = float((lse[fin] - l[fin]).abs().max()) if bool(fin.any()) else 0.0
    return errs
