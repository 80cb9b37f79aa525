"""CPU oracle for the DSA hot path -- TEST INFRASTRUCTURE ONLY.

This package is the checker the HIP kernels are compared against.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it; the product path (``dsa_amd``) never does and
fails loudly when its HIP library is missing.

The arithmetic lives in ``dsa_oracle.c`` (built by ``build_oracle.sh`` into
``libdsa_oracle.so``); this module is a numpy/ctypes front end.  Each
function names the reference code it restates:

* :func:`attention` -- ``solution/triton/indexer_kernel.py:436-497`` (``run()``)
* :func:`e4m3_decode` -- OCP e4m3fn decode used by the indexer
* :func:`indexer_scores` -- score structure of ``indexer_kernel.py:185-275``
  with the exact rounding order documented in ``dsa_oracle.c``
* :func:`topk` -- the selection ``indexer_kernel.py:289-343`` intends
  (score desc, ties to the lower index)
* :func:`e4m3_encode`, :func:`quantize_k`, :func:`pack_k_cache` -- the
  quantise-on-append into the paged fp8 K cache whose records
  ``indexer_kernel.py:163-197`` reads (the reference has no quantisation
  kernel; the formula is the one ``include/dsa_abi.h`` documents)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libdsa_oracle.so")
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build() -> None:
    """Compile ``dsa_oracle.c`` (gcc, no GPU needed)."""
    subprocess.check_call(["sh", os.path.join(_HERE, "build_oracle.sh")])


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        lib.oracle_dsa_attention.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                             _I64, ctypes.c_float, _P, _P, ctypes.c_int]
        lib.oracle_dsa_attention.restype = ctypes.c_int
        lib.oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        lib.oracle_e4m3_decode.restype = ctypes.c_float
        lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
        lib.oracle_indexer_scores.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P,
                                              ctypes.c_int]
        lib.oracle_indexer_scores.restype = ctypes.c_int
        lib.oracle_topk.argtypes = [_P, _P, _I64, _I64, _I64, _P]
        lib.oracle_topk.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=dtype)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 values."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (NaN kept)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def attention(q_nope_bits, q_pe_bits, ckv_bits, kpe_bits, sparse_indices, sm_scale,
              nthreads: int = 0):
    """Restatement of ``run()`` (``indexer_kernel.py:436-497``) in fp64.

    Inputs are bf16 bit patterns (uint16): ``q_nope [T,H,Dc]``, ``q_pe [T,H,Dp]``,
    ``ckv [..., Dc]`` and ``kpe [..., Dp]`` (any paged view; flattened to slots),
    ``sparse_indices [T,K]`` int32 slot ids with -1 padding.
    Returns ``(out_bits [T,H,Dc] uint16, lse [T,H] float32 base-2)``.
    """
    qn = _c(q_nope_bits, np.uint16)
    qp = _c(q_pe_bits, np.uint16)
    T, H, Dc = qn.shape
    Dp = qp.shape[-1]
    kc = _c(ckv_bits, np.uint16).reshape(-1, Dc)
    kp = _c(kpe_bits, np.uint16).reshape(-1, Dp) if Dp else np.zeros((kc.shape[0], 0), np.uint16)
    idx = _c(sparse_indices, np.int32).reshape(T, -1)
    K = idx.shape[1]
    out = np.empty((T, H, Dc), np.uint16)
    lse = np.empty((T, H), np.float32)
    rc = _load().oracle_dsa_attention(_ptr(qn), _ptr(qp), _ptr(kc), _ptr(kp), _ptr(idx), T, H, K,
                                      Dc, Dp, kc.shape[0], float(sm_scale), _ptr(out), _ptr(lse),
                                      int(nthreads))
    if rc != 0:
        raise ValueError(f"oracle_dsa_attention failed (status {rc}): slot id out of range")
    return out, lse


def e4m3_decode(codes) -> np.ndarray:
    """Decode e4m3fn bytes to float32 (table built by the C oracle)."""
    lib = _load()
    table = np.array([lib.oracle_e4m3_decode(i) for i in range(256)], np.float32)
    return table[np.asarray(codes, dtype=np.uint8)]


def indexer_scores(q_codes, k_codes, k_scale, weights, limit, nthreads: int = 0) -> np.ndarray:
    """Exact lightning-indexer scores ``[T,S]`` float32 (masked entries -inf)."""
    q = _c(q_codes, np.uint8)
    k = _c(k_codes, np.uint8)
    T, Hi, D = q.shape
    S = k.shape[0]
    sc = _c(k_scale, np.float32)
    w = _c(weights, np.float32)
    lim = _c(limit, np.int64)
    out = np.empty((T, S), np.float32)
    rc = _load().oracle_indexer_scores(_ptr(q), _ptr(k), _ptr(sc), _ptr(w), _ptr(lim), T, Hi, D,
                                       S, _ptr(out), int(nthreads))
    if rc != 0:
        raise ValueError(f"oracle_indexer_scores failed (status {rc})")
    return out


def topk(scores, limit, k: int) -> np.ndarray:
    """Top-k positions per row, rank order (score desc, position asc), -1 padded."""
    sc = _c(scores, np.float32)
    T, S = sc.shape
    lim = _c(limit, np.int64)
    out = np.empty((T, k), np.int32)
    rc = _load().oracle_topk(_ptr(sc), _ptr(lim), T, S, int(k), _ptr(out))
    if rc != 0:
        raise ValueError(f"oracle_topk failed (status {rc})")
    return out


def e4m3_encode(y) -> np.ndarray:
    """float32 -> e4m3fn codes: the nearest finite e4m3fn value (found by
    search over the 127 non-negative codes, in ascending value order), ties
    to the even code; the sign bit copied (so -0.0 -> 0x80).  |y| <= 448."""
    y = np.asarray(y, dtype=np.float32)
    mag = np.abs(y)
    vals = e4m3_decode(np.arange(0x7f))            # codes 0x00..0x7e, ascending
    hi = np.clip(np.searchsorted(vals, mag, side="left"), 0, len(vals) - 1)
    lo = np.clip(hi - 1, 0, len(vals) - 1)
    d_lo = np.abs(mag - vals[lo])
    d_hi = np.abs(vals[hi] - mag)
    pick = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    return (pick.astype(np.uint8) | np.where(np.signbit(y), 0x80, 0).astype(np.uint8)).astype(np.uint8)


def quantize_k(k) -> tuple:
    """Quantise rows ``k [n, 128]`` (float32 values, e.g. bf16 inputs) with one
    fp32 scale per row: ``scale = fl32(fmax(amax, 1e-4) / 448)``, ``code =
    e4m3_encode(fmin(fmax(fl32(k / scale), -448), 448))`` (fmax/fmin ignore
    NaN).  Returns ``(codes uint8 [n, 128], scale float32 [n])``."""
    k = np.asarray(k, dtype=np.float32)
    amax = np.fmax.reduce(np.abs(k), axis=1).astype(np.float32)
    scale = (np.fmax(amax, np.float32(1e-4)) / np.float32(448.0)).astype(np.float32)
    y = (k / scale[:, None]).astype(np.float32)
    y = np.fmin(np.fmax(y, np.float32(-448.0)), np.float32(448.0)).astype(np.float32)
    return e4m3_encode(y), scale


def pack_k_cache(cache, codes, scale, slots, page_size: int) -> np.ndarray:
    """Write rows into a paged fp8 K cache ``uint8 [pages, page_size * 132]``
    (a copy of ``cache`` is returned): per page the ``page_size x 128`` codes,
    then the ``page_size`` fp32 scales; slot = page * page_size + offset;
    negative or out-of-range slots are skipped."""
    out = np.array(cache, dtype=np.uint8, copy=True)
    pages = out.shape[0]
    sc_bytes = np.asarray(scale, dtype=np.float32).view(np.uint8).reshape(-1, 4)
    for i, sl in enumerate(np.asarray(slots).tolist()):
        if sl < 0 or sl >= pages * page_size:
            continue
        pg, off = divmod(sl, page_size)
        out[pg, off * 128:(off + 1) * 128] = codes[i]
        base = page_size * 128 + off * 4
        out[pg, base:base + 4] = sc_bytes[i]
    return out


def unpack_k_cache(cache, page_size: int, slots) -> tuple:
    """Codes ``[n, 128]`` and scales ``[n]`` of the given slots of a paged cache."""
    cache = np.asarray(cache, dtype=np.uint8)
    slots = np.asarray(slots, dtype=np.int64)
    pg, off = slots // page_size, slots % page_size
    rows = cache[pg[:, None], off[:, None] * 128 + np.arange(128)[None, :]]
    sb = cache[pg[:, None], page_size * 128 + off[:, None] * 4 + np.arange(4)[None, :]]
    return rows, np.ascontiguousarray(sb).view(np.float32).reshape(-1)
