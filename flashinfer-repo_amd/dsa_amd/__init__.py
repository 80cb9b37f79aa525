"""dsa_amd -- MI355X (gfx950) DeepSeek sparse attention hot path.

Hand-written HIP kernels behind a C ABI (``include/dsa_abi.h``,
``libdsa_amd.so``) with a host-side mirror of the reference's entry points:

* ``dsa_amd.kernel``: ``kernel``, ``kernel_splitk``, ``kernel_splitk_v2``,
  ``kernel_out`` (reference ``solution/triton/kernel.py``) and
  ``kernel_noalloc`` (no device allocation: a library-owned scratch array)
* ``dsa_amd.indexer_kernel``: ``run_indexer_and_topk`` (flat or paged fp8 K
  cache, or prepared K planes), ``k_append`` (quantise-on-append into the
  paged cache), ``prepare_k`` / ``prepare_k_paged`` (K operand planes kept
  beside the cache) and the pipeline (reference
  ``solution/triton/indexer_kernel.py``)
* ``dsa_amd.workloads``: seeded synthetic inputs for the benchmark configs
* ``dsa_amd.trace``: replay of recorded workloads (safetensors index files), as the
  reference's test_splitk_correctness.py does
"""
from .indexer_kernel import (KPlanes, k_append, new_k_cache, prepare_k,  # noqa: F401
                             prepare_k_paged, run_indexer_and_topk, run_indexer_and_topk_paged,
                             run_sparse_attention_pipeline)
from .kernel import (kernel, kernel_noalloc, kernel_out, kernel_partial, kernel_splitk,  # noqa: F401
                     kernel_splitk_v2, merge_partials, new_split_counters, new_workspace,
                     num_splits)

__all__ = ["kernel", "kernel_splitk", "kernel_splitk_v2", "kernel_out", "kernel_noalloc",
           "kernel_partial",
           "merge_partials", "new_split_counters", "new_workspace", "num_splits", "run_indexer_and_topk",
           "run_indexer_and_topk_paged", "k_append", "new_k_cache", "run_sparse_attention_pipeline",
           "KPlanes", "prepare_k", "prepare_k_paged"]
