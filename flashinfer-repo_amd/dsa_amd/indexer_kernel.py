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


# Names the reference's per-sequence entry points take
# (solution/triton/indexer_kernel.py:345-363, solution/triton/kernel.py:184-211)
# and this module's per-token ones do not.
_REFERENCE_ONLY_ARGS = frozenset((
    "q_index_fp8", "k_index_cache_fp8", "seq_lens", "seq_offsets", "batch_size",
    "num_index_heads", "index_head_dim", "kv_cache_num_heads", "head_dim_with_scale",
    "max_num_pages", "num_pages", "BLOCK_TOKENS", "BLOCK_HEADS", "device"))

_LAYOUT_NOTE = (
    "this build's {fn} takes the per-query-token layout, not the reference's "
    "per-sequence one (solution/triton/{ref}): one indexer row per query token "
    "(q_idx [T, heads, 128] e4m3fn), k_idx [S, 128] e4m3fn codes with a separate "
    "float32 k_scale [S] (or a paged K cache, see run_indexer_and_topk_paged) instead "
    "of the flat cache of 129-element records, and causal_limit [T] int32 (position s "
    "is a candidate iff s <= causal_limit[t]) instead of seq_lens/seq_offsets/"
    "batch_size.  A sequence b of the reference maps to one row with "
    "causal_limit = seq_lens[b] - 1 and block_table[b] as its block table; the "
    "result holds physical slots (or positions), not seq_offsets-based token ids.")


def _reject_reference_layout(fn: str, ref: str, nargs: int, max_args: int, kwargs) -> None:
    extra = sorted(set(kwargs) & _REFERENCE_ONLY_ARGS)
    if nargs > max_args or extra:
        what = (f"got {nargs} positional arguments" if nargs > max_args
                else f"got reference-only argument(s) {', '.join(extra)}")
        raise TypeError(f"{fn}(): {what}; " + _LAYOUT_NOTE.format(fn=fn, ref=ref))
    unknown = sorted(set(kwargs) - _REFERENCE_ONLY_ARGS)
    if unknown:
        raise TypeError(f"{fn}() got unexpected keyword argument(s) {', '.join(unknown)}")


def run_indexer_and_topk(*args, **kwargs):
    """Top-``topk`` positions (or slots) per query token.

    ``run_indexer_and_topk(q_idx, k_idx, k_scale, weights, causal_limit, topk,
    block_table=None, page_size=64, return_scores=False)``.

    ``score[t,s] = sum_h weights[t,h] * relu(q_idx[t,h] . k_idx[s] * k_scale[s])``
    for ``s <= causal_limit[t]`` (exact rounding order: see ``include/dsa_abi.h``).
    Returns ``int32 [T, topk]`` in ascending position order, -1 padded when a
    row has fewer candidates.  With ``block_table`` (``[T, pages]`` per token,
    or ``[pages]`` shared by all tokens) the entries are physical slots
    ``block_table[page] * page_size + offset``.  With ``return_scores`` the
    fp32 ``[T, S]`` scores (masked entries -inf) are returned too.

    With ``k_planes`` (a :class:`KPlanes` from :func:`prepare_k` or
    :func:`prepare_k_paged`) the call reads the prepared K operand planes
    instead of deriving them from ``k_idx``/``k_scale`` (which may then be
    None; the sequence length is the planes' ``num_positions``); the results
    are the same bits.

    Calls with the reference's per-sequence argument list
    (``indexer_kernel.py:345-363``) raise ``TypeError`` naming the layout
    difference.
    """
    names = ("q_idx", "k_idx", "k_scale", "weights", "causal_limit", "topk", "block_table",
             "page_size", "return_scores", "k_planes")
    mine = {k: kwargs.pop(k) for k in names if k in kwargs}
    _reject_reference_layout("run_indexer_and_topk", "indexer_kernel.py:345-363", len(args),
                             len(names), kwargs)
    bound = dict(zip(names, args))
    for k, v in mine.items():
        if k in bound:
            raise TypeError(f"run_indexer_and_topk() got multiple values for argument {k!r}")
        bound[k] = v
    missing = [k for k in names[:6] if k not in bound]
    if missing:
        raise TypeError(f"run_indexer_and_topk() missing required argument(s) {', '.join(missing)}")
    return _run_indexer_and_topk(**bound)


def _run_indexer_and_topk(q_idx: torch.Tensor, k_idx: Optional[torch.Tensor],
                          k_scale: Optional[torch.Tensor], weights: torch.Tensor,
                          causal_limit: torch.Tensor, topk: int,
                          block_table: Optional[torch.Tensor] = None, page_size: int = 64,
                          return_scores: bool = False, k_planes: Optional["KPlanes"] = None):
    if k_planes is not None:
        _check(isinstance(k_planes, KPlanes), "k_planes must be a KPlanes (see prepare_k)")
        S = k_planes.num_positions
        if k_idx is not None:
            _check(k_idx.shape[0] == S, f"k_idx holds {k_idx.shape[0]} positions, the planes {S}")
        return _indexer(q_idx, S, weights, causal_limit, topk, block_table, page_size,
                        return_scores, planes=k_planes)
    _check(k_idx is not None and k_scale is not None, "k_idx and k_scale are required without k_planes")
    k = _codes(k_idx, "k_idx")
    _check(k.dim() == 2 and k.shape[1] == INDEX_HEAD_DIM,
           f"k_idx must be [S, {INDEX_HEAD_DIM}], got {tuple(k.shape)}")
    S = k.shape[0]
    scale = k_scale.contiguous()
    _check(tuple(scale.shape) == (S,) and scale.dtype == torch.float32, "k_scale must be [S] float32")
    return _indexer(q_idx, S, weights, causal_limit, topk, block_table, page_size, return_scores,
                    flat=(k, scale))


def run_indexer_and_topk_paged(q_idx: torch.Tensor, k_cache: torch.Tensor, k_pages: torch.Tensor,
                               num_positions: int, weights: torch.Tensor,
                               causal_limit: torch.Tensor, topk: int,
                               block_table: Optional[torch.Tensor] = None, page_size: int = 64,
                               return_scores: bool = False):
    """:func:`run_indexer_and_topk` over a paged fp8 K cache (the format
    :func:`k_append` writes): position ``s < num_positions`` is token
    ``s % kps`` of page ``k_pages[s // kps]``, ``kps`` being the cache's page
    size.  The results equal those of the flat call on the same codes and
    scales, bit for bit."""
    cache, kps = _k_cache_view(k_cache)
    pages = k_pages.contiguous()
    S = int(num_positions)
    _check(S >= 0, "num_positions must be >= 0")
    _check(pages.dtype == torch.int32 and pages.dim() == 1 and pages.numel() * kps >= S,
           f"k_pages must be int32 [>= {-(-S // kps)}]")
    return _indexer(q_idx, S, weights, causal_limit, topk, block_table, page_size, return_scores,
                    paged=(cache, pages, kps))


def _indexer(q_idx, S, weights, causal_limit, topk, block_table, page_size, return_scores,
             flat=None, paged=None, planes=None):
    q = _codes(q_idx, "q_idx")
    _check(q.dim() == 3 and q.shape[2] == INDEX_HEAD_DIM,
           f"q_idx must be [T, heads, {INDEX_HEAD_DIM}], got {tuple(q.shape)}")
    T, Hi, _ = q.shape
    _check(Hi in (16, 32, 48, 64), f"index heads must be 16, 32, 48 or 64, got {Hi}")
    dev = q.device
    _check(dev.type == "cuda", "tensors must live on a GPU device")
    w = weights.contiguous()
    lim = causal_limit.contiguous()
    _check(tuple(w.shape) == (T, Hi) and w.dtype == torch.float32, "weights must be [T, heads] float32")
    _check(tuple(lim.shape) == (T,) and lim.dtype == torch.int32, "causal_limit must be [T] int32")
    _check(int(topk) >= 0, "topk must be >= 0")
    held = [x for x in (flat or paged or (planes.buf,)) if isinstance(x, torch.Tensor)]
    for name, x in [("weights", w), ("causal_limit", lim)] + [("k", x) for x in held]:
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
        need = -(-S // int(page_size))
        _check(bt.shape[-1] >= need,
               f"block_table rows hold {bt.shape[-1]} pages; {S} positions of page size "
               f"{int(page_size)} need {need}")

    lib = _lib.load()
    out = torch.empty((T, int(topk)), dtype=torch.int32, device=dev)
    scores = torch.empty((T, S), dtype=torch.float32, device=dev) if return_scores else None
    if planes is not None:
        ws_bytes = lib.dsa_indexer_workspace_bytes_prepared(T, Hi, INDEX_HEAD_DIM, S)
    else:
        ws_bytes = lib.dsa_indexer_workspace_bytes(T, Hi, INDEX_HEAD_DIM, S)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    a = _lib.IndexerArgs()
    a.q_idx, a.weights = q.data_ptr(), w.data_ptr()
    if planes is not None:
        a.k_planes, a.k_planes_capacity = planes.buf.data_ptr(), planes.capacity
    elif flat is not None:
        a.k_idx, a.k_scale = flat[0].data_ptr(), flat[1].data_ptr()
    else:
        a.k_cache, a.k_pages, a.k_page_size = paged[0].data_ptr(), paged[1].data_ptr(), paged[2]
        a.k_num_pages = paged[0].shape[0]
    a.causal_limit = lim.data_ptr()
    a.num_tokens, a.num_heads, a.head_dim, a.num_positions, a.topk = T, Hi, INDEX_HEAD_DIM, S, int(topk)
    a.block_table = bt.data_ptr() if bt is not None else None
    a.block_table_stride, a.page_size = bt_stride, int(page_size)
    a.block_table_width = bt.shape[-1] if bt is not None else 0
    a.out = out.data_ptr() if topk else None
    a.scores_out = scores.data_ptr() if scores is not None else None
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check("dsa_indexer_topk", lib.dsa_indexer_topk(ctypes.byref(a), _stream_handle(dev)))
    return (out, scores) if return_scores else out


class KPlanes:
    """MFMA operand planes of an indexer K sequence, kept beside the K cache
    (``dsa_indexer_prepare_k``): per 16-position block the e4m3 values as
    signed 7-bit pieces in MFMA lane order and the block's largest magnitude,
    and ``fl32(k_scale * 2^-18)`` per position, for up to ``capacity``
    positions.  ``num_positions`` is the sequence length the planes were last
    prepared for.  Made by :func:`prepare_k` / :func:`prepare_k_paged`, which
    also refresh positions of an existing object after an append; pass it to
    :func:`run_indexer_and_topk` as ``k_planes``."""

    def __init__(self, capacity: int, device):
        _check(int(capacity) >= 0, "capacity must be >= 0")
        self.capacity = int(capacity)
        nbytes = _lib.load().dsa_indexer_k_planes_bytes(self.capacity)
        # 256-byte aligned: the caching allocator's blocks start at 512-byte boundaries
        self.buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _check(self.buf.data_ptr() % 256 == 0, "planes buffer is not 256-byte aligned")
        self.num_positions = 0


def _planes_for(planes, S, capacity, dev):
    if planes is None:
        planes = KPlanes(S if capacity is None else capacity, dev)
    _check(isinstance(planes, KPlanes), "planes must be a KPlanes")
    _check(planes.capacity >= S, f"the planes hold {planes.capacity} positions, {S} needed")
    _check(planes.buf.device == dev, f"planes are on {planes.buf.device}, expected {dev}")
    return planes


def _prepare(a, planes, S, first_position, count):
    first = int(first_position)
    n = S - first if count is None else int(count)
    a.num_positions, a.first_position, a.count = S, first, n
    a.k_planes, a.k_planes_capacity = planes.buf.data_ptr(), planes.capacity
    lib = _lib.load()
    _lib.check("dsa_indexer_prepare_k",
               lib.dsa_indexer_prepare_k(ctypes.byref(a), _stream_handle(planes.buf.device)))
    planes.num_positions = S
    return planes


def prepare_k(k_idx: torch.Tensor, k_scale: torch.Tensor, planes: Optional[KPlanes] = None,
              first_position: int = 0, count: Optional[int] = None,
              capacity: Optional[int] = None) -> KPlanes:
    """Derive the K operand planes of ``k_idx [S, 128]`` e4m3fn with
    ``k_scale [S]`` fp32 for positions ``[first_position, first_position +
    count)`` (default: all) -- into ``planes`` when given (e.g. after
    appending positions), else into new planes of ``capacity`` (default S)
    positions.  Returns the planes, now describing S positions."""
    k = _codes(k_idx, "k_idx")
    _check(k.dim() == 2 and k.shape[1] == INDEX_HEAD_DIM,
           f"k_idx must be [S, {INDEX_HEAD_DIM}], got {tuple(k.shape)}")
    S = k.shape[0]
    sc = k_scale.contiguous()
    _check(tuple(sc.shape) == (S,) and sc.dtype == torch.float32, "k_scale must be [S] float32")
    _check(k.device.type == "cuda" and sc.device == k.device, "k_idx and k_scale must be on one GPU")
    planes = _planes_for(planes, S, capacity, k.device)
    a = _lib.KPrepareArgs()
    a.k_idx, a.k_scale = k.data_ptr(), sc.data_ptr()
    return _prepare(a, planes, S, first_position, count)


def prepare_k_paged(k_cache: torch.Tensor, k_pages: torch.Tensor, num_positions: int,
                    planes: Optional[KPlanes] = None, first_position: int = 0,
                    count: Optional[int] = None, capacity: Optional[int] = None) -> KPlanes:
    """:func:`prepare_k` over a paged fp8 K cache (the format :func:`k_append`
    writes), position ``s`` being token ``s % kps`` of page ``k_pages[s //
    kps]``: after ``k_append`` of new positions, ``prepare_k_paged(cache,
    pages, new_length, planes, first_position=old_length)`` refreshes only
    the blocks the append touched."""
    cache, kps = _k_cache_view(k_cache)
    pages = k_pages.contiguous()
    S = int(num_positions)
    _check(S >= 0, "num_positions must be >= 0")
    _check(pages.dtype == torch.int32 and pages.dim() == 1 and pages.numel() * kps >= S,
           f"k_pages must be int32 [>= {-(-S // kps)}]")
    _check(pages.device == cache.device and cache.device.type == "cuda",
           "k_cache and k_pages must be on one GPU")
    planes = _planes_for(planes, S, capacity, cache.device)
    a = _lib.KPrepareArgs()
    a.k_cache, a.k_pages, a.k_page_size = cache.data_ptr(), pages.data_ptr(), kps
    a.k_num_pages = cache.shape[0]
    return _prepare(a, planes, S, first_position, count)


K_TOKEN_BYTES = INDEX_HEAD_DIM + 4  # e4m3 codes + fp32 scale per token


def new_k_cache(num_pages: int, page_size: int, device) -> torch.Tensor:
    """An empty paged fp8 indexer K cache ``uint8 [num_pages, page_size * 132]``:
    per page the ``page_size x 128`` e4m3fn codes, then the ``page_size`` fp32
    scales."""
    _check(int(page_size) > 0 and int(page_size) % 4 == 0, "page_size must be a multiple of 4")
    return torch.zeros((int(num_pages), int(page_size) * K_TOKEN_BYTES), dtype=torch.uint8,
                       device=device)


def _k_cache_view(k_cache: torch.Tensor):
    _check(k_cache.dtype == torch.uint8 and k_cache.dim() == 2
           and k_cache.shape[1] % K_TOKEN_BYTES == 0 and k_cache.is_contiguous(),
           "k_cache must be a contiguous uint8 [pages, page_size * 132] tensor (see new_k_cache)")
    kps = k_cache.shape[1] // K_TOKEN_BYTES
    _check(kps % 4 == 0, "the K cache page size must be a multiple of 4")
    return k_cache, kps


def k_append(k: torch.Tensor, slots: torch.Tensor, k_cache: torch.Tensor) -> torch.Tensor:
    """Quantise bf16 rows ``k [n, 128]`` to e4m3fn with one fp32 scale per row
    (``max(amax, 1e-4) / 448``) and write them to ``slots [n]`` (slot =
    page * page_size + offset; negative slots are skipped) of ``k_cache`` in
    place; returns ``k_cache``."""
    cache, kps = _k_cache_view(k_cache)
    _check(k.dtype == torch.bfloat16 and k.dim() == 2 and k.shape[1] == INDEX_HEAD_DIM,
           f"k must be bfloat16 [n, {INDEX_HEAD_DIM}], got {k.dtype} {tuple(k.shape)}")
    kk = k if (k.stride(1) == 1 and k.stride(0) % 8 == 0 and k.data_ptr() % 16 == 0) else k.contiguous()
    sl = slots.contiguous()
    _check(sl.dtype == torch.int32 and tuple(sl.shape) == (k.shape[0],), "slots must be int32 [n]")
    _check(kk.device == cache.device == sl.device and cache.device.type == "cuda",
           "k, slots and k_cache must live on one GPU device")
    a = _lib.KAppendArgs()
    a.k, a.k_stride, a.slots, a.num_tokens = kk.data_ptr(), kk.stride(0), sl.data_ptr(), kk.shape[0]
    a.k_cache, a.num_pages, a.page_size = cache.data_ptr(), cache.shape[0], kps
    lib = _lib.load()
    _lib.check("dsa_indexer_k_append",
               lib.dsa_indexer_k_append(ctypes.byref(a), _stream_handle(cache.device)))
    return k_cache


_PIPELINE_ARGS = ("q_idx", "k_idx", "k_scale", "weights", "causal_limit", "block_table",
                  "q_nope", "q_pe", "ckv_cache", "kpe_cache", "sm_scale", "topk", "page_size",
                  "k_cache", "k_pages", "num_positions", "k_planes")


def run_sparse_attention_pipeline(*args, **kwargs):
    """Indexer -> top-k slots -> sparse attention, on one stream, no host sync
    (reference ``kernel.py:184-332``).

    ``run_sparse_attention_pipeline(q_idx, k_idx, k_scale, weights,
    causal_limit, block_table, q_nope, q_pe, ckv_cache, kpe_cache, sm_scale,
    topk=2048, page_size=None, k_cache=None, k_pages=None,
    num_positions=None)``.  ``page_size`` defaults to the cache's.
    With ``k_cache`` (a paged fp8 K cache, see :func:`k_append`; ``k_idx`` and
    ``k_scale`` then None) the indexer reads ``num_positions`` positions
    through ``k_pages``, by default the sequence's 1-D ``block_table``; with
    ``k_planes`` (see :func:`prepare_k`) it reads prepared K planes instead.
    Returns ``(output [T,H,512] bf16, lse [T,H] fp32 base-2, slots [T,topk])``.
    Calls with the reference's per-sequence argument list (``kernel.py:184-211``)
    raise ``TypeError`` naming the layout difference."""
    mine = {k: kwargs.pop(k) for k in _PIPELINE_ARGS if k in kwargs}
    _reject_reference_layout("run_sparse_attention_pipeline", "kernel.py:184-211", len(args),
                             len(_PIPELINE_ARGS), kwargs)
    bound = dict(zip(_PIPELINE_ARGS, args))
    for k, v in mine.items():
        if k in bound:
            raise TypeError(f"run_sparse_attention_pipeline() got multiple values for argument {k!r}")
        bound[k] = v
    missing = [k for k in _PIPELINE_ARGS[:11] if k not in bound]
    if missing:
        raise TypeError("run_sparse_attention_pipeline() missing required argument(s) "
                        + ", ".join(missing))
    return _pipeline(**bound)


def _pipeline(q_idx, k_idx, k_scale, weights, causal_limit, block_table, q_nope, q_pe, ckv_cache,
              kpe_cache, sm_scale, topk: int = 2048, page_size: Optional[int] = None,
              k_cache: Optional[torch.Tensor] = None, k_pages: Optional[torch.Tensor] = None,
              num_positions: Optional[int] = None, k_planes: Optional[KPlanes] = None):
    ps = int(page_size) if page_size is not None else (ckv_cache.shape[1] if ckv_cache.dim() == 3 else 1)
    if k_planes is not None:
        slots = _run_indexer_and_topk(q_idx, k_idx, k_scale, weights, causal_limit, topk,
                                      block_table=block_table, page_size=ps, k_planes=k_planes)
    elif k_cache is not None:
        _check(k_idx is None and k_scale is None, "give k_idx/k_scale or k_cache, not both")
        pages = k_pages if k_pages is not None else block_table
        _check(pages is not None and pages.dim() == 1,
               "k_pages (or a 1-D block_table) must map positions to K-cache pages")
        _check(num_positions is not None, "num_positions is required with k_cache")
        slots = run_indexer_and_topk_paged(q_idx, k_cache, pages, int(num_positions), weights,
                                           causal_limit, topk, block_table=block_table, page_size=ps)
    else:
        slots = _run_indexer_and_topk(q_idx, k_idx, k_scale, weights, causal_limit, topk,
                                      block_table=block_table, page_size=ps)
    out, lse = kernel(q_nope, q_pe, ckv_cache, kpe_cache, slots, sm_scale)
    return out, lse, slots
