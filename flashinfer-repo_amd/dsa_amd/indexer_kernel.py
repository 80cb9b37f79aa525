"""Host-side lightning indexer + top-k and the indexer -> attention pipeline.

Counterparts of the reference's ``solution/triton/indexer_kernel.py``
``run_indexer_and_topk`` (:345-433) and ``solution/triton/kernel.py``
``run_sparse_attention_pipeline`` (:184-332), on the per-query-token layout of
the BASELINE indexer workload rather than the reference's per-sequence one:

* one indexer row per query token (the reference scores one query per
  sequence and broadcasts its picks to every token with ``repeat_interleave``
  over KV lengths, ``kernel.py:308-311``);
* ``q_idx [T, Hi, 128]`` and ``k_idx [S, 128]`` e4m3fn with a separate fp32
  ``k_scale [S]`` (the reference stores the scale inline as a 129th element,
  ``indexer_kernel.py:163-197``);
* a causal limit per token instead of ``seq_lens``/``seq_offsets``, and an
  optional block table that turns selected positions into physical cache
  slots inside the top-k kernel, with no host synchronisation (the reference
  reads ``.item()`` twice, ``indexer_kernel.py:371,384``);
* the top-k really selects the k largest scores, ties to the lower position
  (the reference's ``topk_kernel`` collapses to the arg-max,
  ``indexer_kernel.py:330-339``).

Everything runs through ``dsa_indexer_topk`` of the C ABI; shape or dtype
errors raise ``ValueError`` before anything is enqueued.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .kernel import _check, _stream_handle, kernel

INDEX_HEAD_DIM = 128


def _codes(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dtype == torch.float8_e4m3fn:
        x = x.view(torch.uint8)
    _check(x.dtype == torch.uint8, f"{name} must be float8_e4m3fn (or its uint8 codes)")
    return x.contiguous()


def run_indexer_and_topk(q_idx: torch.Tensor, k_idx: torch.Tensor, k_scale: torch.Tensor,
                         weights: torch.Tensor, causal_limit: torch.Tensor, topk: int,
                         block_table: Optional[torch.Tensor] = None, page_size: int = 64,
                         return_scores: bool = False):
    """Top-``topk`` positions (or slots) per query token.

    ``score[t,s] = sum_h weights[t,h] * relu(q_idx[t,h] . k_idx[s] * k_scale[s])``
    for ``s <= causal_limit[t]`` (exact rounding order: see ``include/dsa_abi.h``).
    Returns ``int32 [T, topk]`` in ascending position order, -1 padded when a
    row has fewer candidates.  With ``block_table`` (``[T, pages]`` per token,
    or ``[pages]`` shared by all tokens) the entries are physical slots
    ``block_table[page] * page_size + offset``.  With ``return_scores`` the
    fp32 ``[T, S]`` scores (masked entries -inf) are returned too.
    """
    q = _codes(q_idx, "q_idx")
    k = _codes(k_idx, "k_idx")
    _check(q.dim() == 3 and q.shape[2] == INDEX_HEAD_DIM,
           f"q_idx must be [T, heads, {INDEX_HEAD_DIM}], got {tuple(q.shape)}")
    T, Hi, _ = q.shape
    _check(k.dim() == 2 and k.shape[1] == INDEX_HEAD_DIM,
           f"k_idx must be [S, {INDEX_HEAD_DIM}], got {tuple(k.shape)}")
    S = k.shape[0]
    _check(Hi in (16, 32, 48, 64), f"index heads must be 16, 32, 48 or 64, got {Hi}")
    dev = q.device
    _check(dev.type == "cuda", "tensors must live on a GPU device")
    scale = k_scale.contiguous()
    w = weights.contiguous()
    lim = causal_limit.contiguous()
    _check(tuple(scale.shape) == (S,) and scale.dtype == torch.float32, "k_scale must be [S] float32")
    _check(tuple(w.shape) == (T, Hi) and w.dtype == torch.float32, "weights must be [T, heads] float32")
    _check(tuple(lim.shape) == (T,) and lim.dtype == torch.int32, "causal_limit must be [T] int32")
    _check(int(topk) >= 0, "topk must be >= 0")
    for name, x in (("k_idx", k), ("k_scale", scale), ("weights", w), ("causal_limit", lim)):
        _check(x.device == dev, f"{name} is on {x.device}, expected {dev}")
    bt = None
    bt_stride = 0
    if block_table is not None:
        bt = block_table.contiguous()
        _check(bt.dtype == torch.int32 and bt.device == dev, "block_table must be int32 on the device")
        _check(int(page_size) > 0, "page_size must be > 0")
        if bt.dim() == 1:
            bt_stride = 0
        else:
            _check(bt.dim() == 2 and bt.shape[0] == T, f"block_table must be [{T}, pages] or [pages]")
            bt_stride = bt.stride(0)

    lib = _lib.load()
    out = torch.empty((T, int(topk)), dtype=torch.int32, device=dev)
    scores = torch.empty((T, S), dtype=torch.float32, device=dev) if return_scores else None
    ws_bytes = lib.dsa_indexer_workspace_bytes(T, Hi, INDEX_HEAD_DIM, S)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    a = _lib.IndexerArgs()
    a.q_idx, a.k_idx, a.k_scale, a.weights = q.data_ptr(), k.data_ptr(), scale.data_ptr(), w.data_ptr()
    a.causal_limit = lim.data_ptr()
    a.num_tokens, a.num_heads, a.head_dim, a.num_positions, a.topk = T, Hi, INDEX_HEAD_DIM, S, int(topk)
    a.block_table = bt.data_ptr() if bt is not None else None
    a.block_table_stride, a.page_size = bt_stride, int(page_size)
    a.out = out.data_ptr() if topk else None
    a.scores_out = scores.data_ptr() if scores is not None else None
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check("dsa_indexer_topk", lib.dsa_indexer_topk(ctypes.byref(a), _stream_handle(dev)))
    return (out, scores) if return_scores else out


def run_sparse_attention_pipeline(q_idx, k_idx, k_scale, weights, causal_limit, block_table,
                                  q_nope, q_pe, ckv_cache, kpe_cache, sm_scale, topk: int = 2048,
                                  page_size: Optional[int] = None):
    """Indexer -> top-k slots -> sparse attention, on one stream, no host sync
    (reference ``kernel.py:184-332``).  ``page_size`` defaults to the cache's.
    Returns ``(output [T,H,512] bf16, lse [T,H] fp32 base-2, slots [T,topk])``."""
    ps = int(page_size) if page_size is not None else (ckv_cache.shape[1] if ckv_cache.dim() == 3 else 1)
    slots = run_indexer_and_topk(q_idx, k_idx, k_scale, weights, causal_limit, topk,
                                 block_table=block_table, page_size=ps)
    out, lse = kernel(q_nope, q_pe, ckv_cache, kpe_cache, slots, sm_scale)
    return out, lse, slots
