"""The allocation-free entry point dsa_attn_fwd_noalloc against dsa_attn_fwd.

dsa_attn_fwd_noalloc has no counterpart in the reference: it is the
attention call for callers that cannot allocate device memory, with the
split partials in the library's per-device scratch array.  Its results must
equal dsa_attn_fwd's bit for bit (both merge the splits in the same order
with the same arithmetic), on consecutive calls that reuse the array, the
second with a smaller input, and both must be within the reference checker's
tolerance of the CPU oracle.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, mismatches
from dsa_amd import _lib, kernel_out, kernel_noalloc, workloads

DEV = "cuda:0"
NTHREADS = min(16, os.cpu_count() or 1)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.gpu
def test_noalloc_equals_dsa_attn_fwd_on_consecutive_calls():
    # (T, splits, seed); T=64 has 4 splits, which kernel_out merges inside the
    # attention kernel (the others, and every no-alloc call, use the merge kernel)
    cases = [(48, 0, 901), (48, 7, 902), (5, 0, 903), (3, 16, 904), (64, 0, 906)]
    for T, splits, seed in cases:
        d = workloads.cfg2(T=T, seed=seed)
        g = workloads.to_device(d, DEV)
        args = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], g["sparse_indices"],
                d["sm_scale"])
        print(f"noalloc T={T} splits={splits}", flush=True)
        out_n = torch.full((T, 16, 512), 7.0, dtype=torch.bfloat16, device=DEV)
        lse_n = torch.full((T, 16), 7.0, dtype=torch.float32, device=DEV)
        torch.cuda.synchronize()
        kernel_noalloc(*args, out_n, lse_n, num_splits=splits)
        out_r = torch.empty_like(out_n)
        lse_r = torch.empty_like(lse_n)
        kernel_out(*args, out_r, lse_r, num_splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(out_n, out_r) and torch.equal(lse_n, lse_r), (T, splits)
        ref_bits, ref_lse = oracle.attention(_bits(d["q_nope"]), _bits(d["q_pe"]),
                                             _bits(d["ckv_cache"]), _bits(d["kpe_cache"]),
                                             d["sparse_indices"].numpy(), d["sm_scale"], NTHREADS)
        assert mismatches(out_n.float().cpu().numpy(), oracle.bf16_bits_to_f32(ref_bits),
                          OUT_ATOL, OUT_RTOL) == 0
        assert mismatches(lse_n.cpu().numpy(), ref_lse, LSE_ATOL, LSE_RTOL) == 0


@pytest.mark.gpu
def test_noalloc_rejects_workspace_beyond_the_scratch_array():
    lib = _lib.load()
    d = workloads.cfg2(T=2, seed=905)
    g = workloads.to_device(d, DEV)
    T, K = 600, 2048
    need = lib.dsa_attn_workspace_bytes(T, 16, K, 8)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    q = g["q_nope"][:1].expand(T, 16, 512)
    qp = g["q_pe"][:1].expand(T, 16, 64)
    idx = g["sparse_indices"][:1].expand(T, K)
    out = torch.empty((T, 16, 512), dtype=torch.bfloat16, device=DEV)
    lse = torch.empty((T, 16), dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError, match="scratch array"):
        kernel_noalloc(q, qp, g["ckv_cache"], g["kpe_cache"], idx, d["sm_scale"], out, lse,
                       num_splits=8)


def test_noalloc_host_checks_need_no_device():
    """Size and argument checks happen before any device call."""
    lib = _lib.load()
    a = _lib.AttnArgs()
    a.num_tokens, a.num_heads, a.topk, a.num_splits = 4096, 16, 2048, 4
    a.head_dim_ckv, a.head_dim_kpe, a.page_size = 512, 64, 64
    assert lib.dsa_attn_fwd_noalloc(ctypes.byref(a), None) == _lib.DSA_EWORKSPACE
    assert b"scratch array" in lib.dsa_last_error()
    a.workspace, a.workspace_bytes = 0x1000, 1 << 30
    assert lib.dsa_attn_fwd_noalloc(ctypes.byref(a), None) == _lib.DSA_EINVAL
    assert lib.dsa_attn_fwd_noalloc(None, None) == _lib.DSA_EINVAL
