"""dsa_amd -- MI355X (gfx950) DeepSeek sparse attention hot path.

Hand-written HIP kernels behind a C ABI (``include/dsa_abi.h``,
``libdsa_amd.so``) with a host-side mirror of the reference's entry points:

* ``dsa_amd.kernel``: ``kernel``, ``kernel_splitk``, ``kernel_splitk_v2``,
  ``kernel_out`` (reference ``solution/triton/kernel.py``)
* ``dsa_amd.indexer_kernel``: ``run_indexer_and_topk`` and the pipeline
  (reference ``solution/triton/indexer_kernel.py``)
* ``dsa_amd.workloads``: seeded synthetic inputs for the benchmark configs
"""
from .indexer_kernel import run_indexer_and_topk, run_sparse_attention_pipeline  # noqa: F401
from .kernel import (kernel, kernel_out, kernel_partial, kernel_splitk, kernel_splitk_v2,  # noqa: F401
                     merge_partials, new_split_counters, new_workspace, num_splits)

__all__ = ["kernel", "kernel_splitk", "kernel_splitk_v2", "kernel_out", "kernel_partial",
           "merge_partials", "new_split_counters", "new_workspace", "num_splits", "run_indexer_and_topk",
           "run_sparse_attention_pipeline"]
