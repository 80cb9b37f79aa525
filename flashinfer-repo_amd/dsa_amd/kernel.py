"""Host-side mirror of the reference's DSA attention entry points.

Same names, arguments and return values as ``solution/triton/kernel.py`` of the
reference, so its drivers (``test_splitk_correctness.py``,
``profile_kernel*.py``) run unchanged against this module:

* :func:`kernel`            -- ``kernel.py:138-182``
* :func:`kernel_splitk`     -- ``kernel.py:496-567``
* :func:`kernel_splitk_v2`  -- ``kernel.py:707-799``
* :func:`kernel_out`        -- destination-passing variant (``output``/``lse``
  appended, the flashinfer-bench DPS convention)

All of them call the HIP library through its C ABI (``dsa_attn_fwd``); the
tensors only supply device pointers, strides and the current stream.  The
reference's constant asserts (H=16, page_size=64, topk=2048,
``kernel.py:147-151``) are relaxed to what the kernels implement: any number of
tokens and pages, any page size and top-k, H a multiple of 16, head dims
512/64.  Shape or dtype errors raise ``ValueError`` before anything is
enqueued.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib

HEAD_DIM_CKV = 512
HEAD_DIM_KPE = 64


def _stream_handle(device: torch.device) -> int:
    """The current HIP stream of ``device`` as a raw handle (an int)."""
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None
                                              else torch.cuda.current_device())


def new_workspace(q_nope: torch.Tensor, topk: int, num_splits: int = 0) -> torch.Tensor:
    """A workspace for calls of this shape, for callers that manage their own
    (e.g. to keep allocation out of a serving loop); pass it to
    :func:`kernel_out`.  Its contents do not matter."""
    T, H, _ = q_nope.shape
    nbytes = _lib.load().dsa_attn_workspace_bytes(T, H, topk, int(num_splits))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=q_nope.device)


def new_split_counters(q_nope: torch.Tensor) -> torch.Tensor:
    """Zeroed merge counters for calls of up to ``q_nope``'s token and head
    counts (pass to :func:`kernel_out`).  Calls of head counts with an odd
    number of 16-head groups (e.g. H=16 decode) and 2 to 4 splits that are
    given them merge their chunks inside the attention kernel and leave them
    zero again (other calls ignore them and run the merge kernel); calls that
    may run at the same time (other streams, graphs replayed concurrently)
    each need their own."""
    T, H, _ = q_nope.shape
    nbytes = _lib.load().dsa_attn_counter_bytes(T, H)
    return torch.zeros(max(nbytes // 4, 1), dtype=torch.int32, device=q_nope.device)


# Merge counters of calls that bring none.  Each (device, stream) has two
# zeroed buffers: one for eager calls and one for calls captured into HIP
# graphs on that stream, so a graph replayed while eager calls run on its
# capture stream does not share counters with them.  A call leaves its
# counters zero again, so calls of one stream (and sequential replays) can
# share a buffer.  Buffers are made (and zeroed) outside capture only: a
# captured call that finds no large enough buffer merges with the separate
# merge kernel instead.  A buffer that was ever handed to a call is never
# freed -- a graph keeps its raw address -- so a buffer outgrown by a later
# call is retired, not released.  Replaying two graphs captured on one
# stream at the same time (on different streams) shares their buffer: pass
# split_counters to such graphs.
_stream_counters = {}
_retired_counters = []


def _default_counters(dev: torch.device, nbytes: int) -> Optional[torch.Tensor]:
    capturing = torch.cuda.is_current_stream_capturing()
    handle = _stream_handle(dev)
    key = (dev.index, handle, capturing)
    buf = _stream_counters.get(key)
    if buf is not None and buf.numel() * 4 >= nbytes:
        return buf
    if capturing:
        return None
    words = max(nbytes // 4, 2 * buf.numel() if buf is not None else 0, 4096)
    for k in (key, (dev.index, handle, True)):
        old = _stream_counters.get(k)
        if old is not None and old.numel() >= words:
            continue
        if old is not None:
            _retired_counters.append(old)
        _stream_counters[k] = torch.zeros(words, dtype=torch.int32, device=dev)
    return _stream_counters[key]


def _rezero_counters(cnt: torch.Tensor) -> None:
    """After a call that failed, its counters may not be zero: clear them
    (outside capture; a failed captured call invalidates the capture anyway)."""
    if not torch.cuda.is_current_stream_capturing():
        cnt.zero_()


def _inner_contiguous(x: torch.Tensor) -> torch.Tensor:
    return x if x.stride(-1) == 1 else x.contiguous()


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _cache_view(cache: torch.Tensor, dim: int, name: str) -> Tuple[torch.Tensor, int, int, int, int]:
    """Return (tensor, num_pages, page_size, stride_page, stride_tok) for a
    paged cache ``[pages, page_size, dim]`` or a flat ``[slots, dim]`` one."""
    _check(cache.dtype == torch.bfloat16, f"{name} must be bfloat16, got {cache.dtype}")
    _check(cache.shape[-1] == dim, f"{name} last dim must be {dim}, got {tuple(cache.shape)}")
    cache = _inner_contiguous(cache)
    if cache.dim() == 3:
        return cache, cache.shape[0], cache.shape[1], cache.stride(0), cache.stride(1)
    if cache.dim() == 2:
        return cache, cache.shape[0], 1, cache.stride(0), cache.stride(0)
    raise ValueError(f"{name} must be [pages, page_size, {dim}] or [slots, {dim}]")


def _attn_args(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, num_splits: int):
    """Validate the reference tensor contract (``kernel.py:138-151``) and build
    the ``dsa_attn_args`` struct; returns ``(args, keep_alive, T, H, K, dev)``
    with output/lse/workspace still unset."""
    if isinstance(sm_scale, torch.Tensor):
        _check(sm_scale.numel() == 1, "sm_scale must be a number or a one-element tensor")
        if sm_scale.device.type != "cpu" and torch.cuda.is_current_stream_capturing():
            raise ValueError("sm_scale is a device tensor: reading it needs a device-to-host "
                             "copy, which cannot happen during graph capture; pass a float")
        sm_scale = float(sm_scale.item())
    _check(q_nope.dim() == 3 and q_pe.dim() == 3, "q_nope/q_pe must be [T, H, D]")
    T, H, dc = q_nope.shape
    _check(dc == HEAD_DIM_CKV, f"q_nope head dim must be {HEAD_DIM_CKV}, got {dc}")
    _check(tuple(q_pe.shape) == (T, H, HEAD_DIM_KPE),
           f"q_pe must be [{T}, {H}, {HEAD_DIM_KPE}], got {tuple(q_pe.shape)}")
    _check(q_nope.dtype == torch.bfloat16 and q_pe.dtype == torch.bfloat16,
           "q_nope/q_pe must be bfloat16")
    _check(H % 16 == 0, f"num heads must be a multiple of 16, got {H}")
    _check(sparse_indices.dim() == 2 and sparse_indices.shape[0] == T,
           f"sparse_indices must be [{T}, topk], got {tuple(sparse_indices.shape)}")
    _check(sparse_indices.dtype == torch.int32, "sparse_indices must be int32")
    _check(int(num_splits) >= 0, f"num_splits must be >= 0, got {num_splits}")
    dev = q_nope.device
    _check(dev.type == "cuda", "tensors must live on a GPU device")
    for name, x in (("q_pe", q_pe), ("ckv_cache", ckv_cache), ("kpe_cache", kpe_cache),
                    ("sparse_indices", sparse_indices)):
        _check(x.device == dev, f"{name} is on {x.device}, expected {dev}")
    ckv, pages, ps, ckv_sp, ckv_so = _cache_view(ckv_cache, HEAD_DIM_CKV, "ckv_cache")
    kpe, kpages, kps, kpe_sp, kpe_so = _cache_view(kpe_cache, HEAD_DIM_KPE, "kpe_cache")
    _check((pages, ps) == (kpages, kps), "ckv_cache and kpe_cache page layouts differ")
    q_nope = _inner_contiguous(q_nope)
    q_pe = _inner_contiguous(q_pe)
    idx = _inner_contiguous(sparse_indices)
    K = idx.shape[1]
    a = _lib.AttnArgs()
    a.q_nope, a.q_nope_stride_t, a.q_nope_stride_h = q_nope.data_ptr(), q_nope.stride(0), q_nope.stride(1)
    a.q_pe, a.q_pe_stride_t, a.q_pe_stride_h = q_pe.data_ptr(), q_pe.stride(0), q_pe.stride(1)
    a.ckv, a.ckv_stride_page, a.ckv_stride_tok = ckv.data_ptr(), ckv_sp, ckv_so
    a.kpe, a.kpe_stride_page, a.kpe_stride_tok = kpe.data_ptr(), kpe_sp, kpe_so
    a.sparse_indices, a.idx_stride_t = idx.data_ptr(), idx.stride(0)
    a.num_tokens, a.num_heads, a.topk = T, H, K
    a.page_size, a.num_pages = ps, pages
    a.head_dim_ckv, a.head_dim_kpe = HEAD_DIM_CKV, HEAD_DIM_KPE
    a.sm_scale = float(sm_scale)
    a.num_splits = int(num_splits)
    return a, (q_nope, q_pe, ckv, kpe, idx), T, H, K, dev


# Validated call shapes of the value-returning entry points: a call whose
# tensors have the shapes, strides, dtypes and devices of an earlier one (and
# the same scale and split request) reuses that call's checked argument
# struct and size queries and only sets the data pointers, so an eager call
# costs little more than the launch.  Calls whose tensors would need a copy
# (a non-contiguous last dimension) always take the checked path.
class _Plan:
    __slots__ = ("template", "T", "H", "dev", "ws_bytes", "c_bytes")


_plans = {}
_PLAN_LIMIT = 256

# Workspaces of eager calls that bring none, one grow-only buffer per (device,
# stream): calls of one stream run one after another, and a workspace's
# contents do not matter.  Calls under graph capture take theirs from the
# graph's memory pool instead.
_stream_workspaces = {}


def _plan_key(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, num_splits):
    return (q_nope.shape, q_nope.stride(), q_nope.dtype, q_nope.get_device(),
            q_pe.shape, q_pe.stride(), q_pe.dtype, q_pe.get_device(),
            ckv_cache.shape, ckv_cache.stride(), ckv_cache.dtype, ckv_cache.get_device(),
            kpe_cache.shape, kpe_cache.stride(), kpe_cache.dtype, kpe_cache.get_device(),
            sparse_indices.shape, sparse_indices.stride(), sparse_indices.dtype,
            sparse_indices.get_device(), sm_scale, num_splits)


def _make_plan(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, num_splits):
    """Checks the call (raising as the checked path does) and returns its
    plan, or None when a tensor would need a copy."""
    a, keep, T, H, K, dev = _attn_args(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices,
                                       sm_scale, num_splits)
    if any(x.data_ptr() != y.data_ptr() for x, y in
           zip(keep, (q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices))):
        return None
    lib = _lib.load()
    plan = _Plan()
    a.out_stride_t, a.out_stride_h = H * HEAD_DIM_CKV, HEAD_DIM_CKV
    a.lse_stride_t, a.lse_stride_h = H, 1
    plan.template = bytes(a)
    plan.T, plan.H, plan.dev = T, H, dev
    plan.ws_bytes = lib.dsa_attn_workspace_bytes(T, H, K, int(num_splits))
    # counters only for calls that merge their splits inside the attention
    # kernel (the others run the merge kernel and never touch them)
    plan.c_bytes = lib.dsa_attn_call_counter_bytes(T, H, K, int(num_splits)) if plan.ws_bytes else 0
    return plan


def _stream_workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (dev.index, stream)
    buf = _stream_workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 2 * buf.numel() if buf is not None else 0),
                          dtype=torch.uint8, device=dev)
        _stream_workspaces[key] = buf
    return buf


def _check_output(output, T, H, dev):
    _check(tuple(output.shape) == (T, H, HEAD_DIM_CKV) and output.dtype == torch.bfloat16
           and output.stride(-1) == 1 and output.device == dev,
           "output must be a [T, H, 512] bfloat16 tensor with a contiguous last dim")


def _check_lse(lse, T, H, dev):
    _check(tuple(lse.shape) == (T, H) and lse.dtype == torch.float32 and lse.device == dev,
           "lse must be a [T, H] float32 tensor")


def _check_workspace(workspace, ws_bytes, dev):
    _check(workspace.device == dev and workspace.is_contiguous()
           and workspace.numel() * workspace.element_size() >= ws_bytes,
           f"workspace must be a contiguous tensor of >= {ws_bytes} bytes on {dev}")


def _check_counters(split_counters, c_bytes, dev):
    _check(split_counters.device == dev and split_counters.is_contiguous()
           and split_counters.dtype == torch.int32
           and split_counters.numel() * 4 >= c_bytes,
           f"split_counters must be a contiguous int32 tensor of >= {c_bytes // 4} "
           f"elements on {dev} (see new_split_counters)")


def _attention_planned(plan, q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices,
                       output=None, lse=None, workspace=None, split_counters=None):
    a = _lib.AttnArgs.from_buffer_copy(plan.template)
    a.q_nope, a.q_pe = q_nope.data_ptr(), q_pe.data_ptr()
    a.ckv, a.kpe, a.sparse_indices = ckv_cache.data_ptr(), kpe_cache.data_ptr(), sparse_indices.data_ptr()
    dev = plan.dev
    if output is None:
        output = torch.empty((plan.T, plan.H, HEAD_DIM_CKV), dtype=torch.bfloat16, device=dev)
    else:
        _check_output(output, plan.T, plan.H, dev)
        a.out_stride_t, a.out_stride_h = output.stride(0), output.stride(1)
    if lse is None:
        lse = torch.empty((plan.T, plan.H), dtype=torch.float32, device=dev)
    else:
        _check_lse(lse, plan.T, plan.H, dev)
        a.lse_stride_t, a.lse_stride_h = lse.stride(0), lse.stride(1)
    a.output, a.lse = output.data_ptr(), lse.data_ptr()
    stream = _stream_handle(dev)
    cnt = None
    if plan.ws_bytes:
        if workspace is not None:
            _check_workspace(workspace, plan.ws_bytes, dev)
            ws = workspace
        elif torch.cuda.is_current_stream_capturing():
            ws = torch.empty(plan.ws_bytes, dtype=torch.uint8, device=dev)
        else:
            ws = _stream_workspace(dev, stream, plan.ws_bytes)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * ws.element_size()
        if plan.c_bytes:
            if split_counters is not None:
                _check_counters(split_counters, plan.c_bytes, dev)
                cnt = split_counters
            else:
                cnt = _default_counters(dev, plan.c_bytes)
            if cnt is not None:
                a.split_counters, a.split_counters_bytes = cnt.data_ptr(), cnt.numel() * 4
    lib = _lib.load()
    rc = lib.dsa_attn_fwd(ctypes.byref(a), stream)
    if rc != _lib.DSA_OK and cnt is not None:
        _rezero_counters(cnt)
    _lib.check("dsa_attn_fwd", rc)
    return output, lse


def _attention(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, num_splits: int,
               output: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
               workspace: Optional[torch.Tensor] = None,
               split_counters: Optional[torch.Tensor] = None):
    if isinstance(sm_scale, (int, float)):
        try:
            key = _plan_key(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale,
                            num_splits)
        except (AttributeError, TypeError):
            key = None  # not tensors: the checked path below raises
        if key is not None:
            plan = _plans.get(key)
            if plan is None:
                plan = _make_plan(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale,
                                  num_splits)
                if plan is not None:
                    if len(_plans) >= _PLAN_LIMIT:
                        _plans.clear()
                    _plans[key] = plan
            if plan is not None:
                return _attention_planned(plan, q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices,
                                          output, lse, workspace, split_counters)
    a, keep, T, H, K, dev = _attn_args(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices,
                                       sm_scale, num_splits)
    if output is None:
        output = torch.empty((T, H, HEAD_DIM_CKV), dtype=torch.bfloat16, device=dev)
    if lse is None:
        lse = torch.empty((T, H), dtype=torch.float32, device=dev)
    _check_output(output, T, H, dev)
    _check_lse(lse, T, H, dev)
    lib = _lib.load()
    ws_bytes = lib.dsa_attn_workspace_bytes(T, H, K, int(num_splits))
    ws = None
    if ws_bytes:
        if workspace is not None:
            _check_workspace(workspace, ws_bytes, dev)
            ws = workspace
            ws_bytes = workspace.numel() * workspace.element_size()
        else:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    a.output, a.out_stride_t, a.out_stride_h = output.data_ptr(), output.stride(0), output.stride(1)
    a.lse, a.lse_stride_t, a.lse_stride_h = lse.data_ptr(), lse.stride(0), lse.stride(1)
    a.workspace = ws.data_ptr() if ws is not None else None
    a.workspace_bytes = ws_bytes
    c_bytes = lib.dsa_attn_call_counter_bytes(T, H, K, int(num_splits)) if ws is not None else 0
    if c_bytes:
        if split_counters is not None:
            _check_counters(split_counters, c_bytes, dev)
            cnt = split_counters
        else:
            cnt = _default_counters(dev, c_bytes)
        if cnt is not None:
            a.split_counters, a.split_counters_bytes = cnt.data_ptr(), cnt.numel() * 4
    else:
        cnt = None
    rc = lib.dsa_attn_fwd(ctypes.byref(a), _stream_handle(dev))
    if rc != _lib.DSA_OK and cnt is not None:
        _rezero_counters(cnt)
    _lib.check("dsa_attn_fwd", rc)
    del keep
    return output, lse


def kernel(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale):
    """Sparse MLA attention (reference ``kernel.py:138``).

    Returns ``(output [T,H,512] bf16, lse [T,H] fp32 base-2)``.  The split of
    the top-k axis over workgroups is chosen automatically to fill the GPU.
    """
    return _attention(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, 0)


def kernel_splitk(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, SPLIT_K=16):
    """Split-K variant (reference ``kernel.py:496``): the top-k axis is cut into
    ``SPLIT_K`` chunks computed in parallel and merged with log-sum-exp
    weights.  Unlike the reference, ``topk % SPLIT_K`` need not be 0."""
    _check(int(SPLIT_K) >= 1, f"SPLIT_K must be >= 1, got {SPLIT_K}")
    return _attention(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, int(SPLIT_K))


def kernel_splitk_v2(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, SPLIT_K=16):
    """Reference ``kernel.py:707``: same result as :func:`kernel_splitk`.  The
    reference's three-phase merge with fp32 atomics (``kernel.py:583-704``) is
    replaced by the one deterministic merge kernel."""
    return kernel_splitk(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, SPLIT_K)


def kernel_out(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, output, lse,
               num_splits: int = 0, workspace: Optional[torch.Tensor] = None,
               split_counters: Optional[torch.Tensor] = None):
    """Destination-passing variant: writes into ``output`` and ``lse``.

    ``workspace`` (optional) comes from :func:`new_workspace`; by default one
    is taken from the framework's caching allocator for the call.
    ``split_counters`` (optional) comes from :func:`new_split_counters`; by
    default the calls of one stream share a zeroed buffer kept per stream."""
    _attention(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, int(num_splits),
               output=output, lse=lse, workspace=workspace, split_counters=split_counters)
    return output, lse


def kernel_noalloc(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale, output, lse,
                   num_splits: int = 0):
    """Destination-passing call that allocates nothing (``dsa_attn_fwd_noalloc``):
    split partials go to the library's per-device scratch array
    (``NOALLOC_SCRATCH_BYTES``, 32 MiB) instead of a workspace, and are merged
    by the separate merge kernel.  Inputs must already have contiguous last
    dimensions and 16-byte aligned rows (nothing is copied); a split workspace
    beyond the scratch array raises ``ValueError``.  Calls that overlap on
    one device race on the array."""
    for name, x in (("q_nope", q_nope), ("q_pe", q_pe), ("ckv_cache", ckv_cache),
                    ("kpe_cache", kpe_cache), ("sparse_indices", sparse_indices)):
        _check(x.stride(-1) == 1, f"{name} must have a contiguous last dimension")
    a, keep, T, H, K, dev = _attn_args(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices,
                                       sm_scale, num_splits)
    _check_output(output, T, H, dev)
    _check_lse(lse, T, H, dev)
    a.output, a.out_stride_t, a.out_stride_h = output.data_ptr(), output.stride(0), output.stride(1)
    a.lse, a.lse_stride_t, a.lse_stride_h = lse.data_ptr(), lse.stride(0), lse.stride(1)
    lib = _lib.load()
    _lib.check("dsa_attn_fwd_noalloc", lib.dsa_attn_fwd_noalloc(ctypes.byref(a),
                                                                _stream_handle(dev)))
    del keep
    return output, lse


def kernel_partial(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices, sm_scale,
                   num_splits: int = 0):
    """Per-chunk partials without the merge (the split half of
    ``kernel_splitk``, reference ``kernel.py:343-434``).

    Returns ``(part_acc [T,S,H,512] fp32, part_ml [T,S,H,2] fp32)``: for chunk
    s, ``part_ml[...,0]`` is a reference max m (log2 units), ``part_ml[...,1]``
    the sum of ``2^(x*log2(e) - m)`` over the chunk's valid slots and
    ``part_acc`` the matching weighted sum of ckv rows.  Partials of disjoint
    slot sets (e.g. cache shards on different devices) concatenated along S
    merge with :func:`merge_partials`."""
    a, keep, T, H, K, dev = _attn_args(q_nope, q_pe, ckv_cache, kpe_cache, sparse_indices,
                                       sm_scale, num_splits)
    lib = _lib.load()
    S = int(lib.dsa_attn_num_splits(T, H, K, int(num_splits)))
    nbytes = lib.dsa_attn_partial_bytes(T, H, K, int(num_splits))
    ws = torch.empty(max(nbytes // 4, 4), dtype=torch.float32, device=dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    _lib.check("dsa_attn_fwd_partial", lib.dsa_attn_fwd_partial(ctypes.byref(a),
                                                                _stream_handle(dev)))
    del keep
    n_acc = T * S * H * HEAD_DIM_CKV
    return ws[:n_acc].view(T, S, H, HEAD_DIM_CKV), ws[n_acc:n_acc + T * S * H * 2].view(T, S, H, 2)


def merge_partials(part_acc: torch.Tensor, part_ml: torch.Tensor,
                   output: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None):
    """Log-sum-exp merge of partials along S (reference ``kernel.py:437-493``);
    returns ``(output [T,H,512] bf16, lse [T,H] fp32 base-2)``."""
    _check(part_acc.dim() == 4 and part_acc.shape[-1] == HEAD_DIM_CKV
           and part_acc.dtype == torch.float32, "part_acc must be [T, S, H, 512] float32")
    T, S, H, _ = part_acc.shape
    _check(tuple(part_ml.shape) == (T, S, H, 2) and part_ml.dtype == torch.float32,
           f"part_ml must be [{T}, {S}, {H}, 2] float32")
    _check(part_acc.device == part_ml.device and part_acc.device.type == "cuda",
           "partials must live on one GPU device")
    dev = part_acc.device
    acc = part_acc.contiguous()
    ml = part_ml.contiguous()
    if output is None:
        output = torch.empty((T, H, HEAD_DIM_CKV), dtype=torch.bfloat16, device=dev)
    if lse is None:
        lse = torch.empty((T, H), dtype=torch.float32, device=dev)
    m = _lib.MergeArgs()
    m.part_acc, m.part_ml = acc.data_ptr(), ml.data_ptr()
    m.num_tokens, m.num_splits, m.num_heads = T, S, H
    m.output, m.out_stride_t, m.out_stride_h = output.data_ptr(), output.stride(0), output.stride(1)
    m.lse, m.lse_stride_t, m.lse_stride_h = lse.data_ptr(), lse.stride(0), lse.stride(1)
    lib = _lib.load()
    _lib.check("dsa_attn_merge", lib.dsa_attn_merge(ctypes.byref(m), _stream_handle(dev)))
    return output, lse


def num_splits(num_tokens: int, num_heads: int, topk: int, requested: int = 0) -> int:
    """Split count :func:`kernel` (requested=0) or :func:`kernel_splitk` uses."""
    return int(_lib.load().dsa_attn_num_splits(num_tokens, num_heads, topk, requested))
