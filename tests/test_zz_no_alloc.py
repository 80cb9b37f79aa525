"""The allocation-free entry point dsa_attn_fwd_noalloc against dsa_attn_fwd.

dsa_attn_fwd_noalloc has no counterpart in the reference: it is the
attention call for callers that cannot allocate device memory, with the
split partials in the library's per-device scratch array.  Its results must
equal dsa_attn_fwd's bit for bit (both merge the splits in the same order
with the same arithmetic), on consecutive calls that reuse the array, the
second with a smaller input, and both must be within the reference checker's
tolerance of the CPU oracle.  The first test makes the process's first
no-alloc call inside a HIP graph capture (the call looks up the scratch
array's address on its first use on a device) and replays the graph.
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
SM = workloads.SM_SCALE
NTHREADS = min(16, os.cpu_count() or 1)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _noalloc_splits(T, H, K):
    """The split count an automatic no-alloc call takes: the automatic count
    when its workspace fits the scratch array, else the most splits below it
    that fit (as dsa_attn_fwd_noalloc chooses)."""
    lib = _lib.load()
    if lib.dsa_attn_workspace_bytes(T, H, K, 0) <= _lib.NOALLOC_SCRATCH_BYTES:
        return 0
    for s in range(lib.dsa_attn_num_splits(T, H, K, 0) - 1, 0, -1):
        if lib.dsa_attn_workspace_bytes(T, H, K, s) <= _lib.NOALLOC_SCRATCH_BYTES:
            return s
    raise AssertionError("no split count fits")


# Must stay the first test of this file: it makes the process's first
# no-alloc call, and makes it inside a graph capture.
@pytest.mark.gpu
def test_noalloc_first_call_captured_in_a_graph():
    T = 48  # 5 automatic splits: the partials go to the scratch array
    d = workloads.cfg2(T=T, seed=907)
    g = workloads.to_device(d, DEV)
    args = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], g["sparse_indices"],
            d["sm_scale"])
    assert _lib.load().dsa_attn_workspace_bytes(T, 16, 2048, 0) > 0
    out_n = torch.empty((T, 16, 512), dtype=torch.bfloat16, device=DEV)
    lse_n = torch.empty((T, 16), dtype=torch.float32, device=DEV)
    torch.cuda.synchronize()
    print("noalloc: first call inside graph capture", flush=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        kernel_noalloc(*args, out_n, lse_n)
    torch.cuda.synchronize()
    out_r = torch.empty_like(out_n)
    lse_r = torch.empty_like(lse_n)
    kernel_out(*args, out_r, lse_r)
    torch.cuda.synchronize()
    for r in range(4):
        # eager work on the outputs between replays
        out_n.fill_(7.0)
        lse_n.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_n, out_r) and torch.equal(lse_n, lse_r), f"replay {r}"


@pytest.mark.gpu
def test_noalloc_automatic_splits_reduced_to_fit_the_scratch_array():
    """H=128 T=64 takes 2 automatic splits whose 34.6 MB workspace exceeds the
    array: the no-alloc call runs one split (no workspace) and equals
    dsa_attn_fwd with that count bit for bit."""
    lib = _lib.load()
    T, H, K = 64, 128, 2048
    assert lib.dsa_attn_workspace_bytes(T, H, K, 0) > _lib.NOALLOC_SCRATCH_BYTES
    splits = _noalloc_splits(T, H, K)
    assert splits == 1
    d = workloads.attention_inputs(T, H, K, 1024, 64, seed=908)
    gen = d.pop("gen")
    idx = torch.stack([torch.randperm(1024 * 64, generator=gen)[:K] for _ in range(T)]).to(torch.int32)
    idx[5, 1000:] = -1
    g = workloads.to_device(d, DEV)
    args = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], idx.to(DEV), SM)
    print(f"noalloc H={H} T={T} automatic splits -> {splits}", flush=True)
    out_n = torch.empty((T, H, 512), dtype=torch.bfloat16, device=DEV)
    lse_n = torch.empty((T, H), dtype=torch.float32, device=DEV)
    kernel_noalloc(*args, out_n, lse_n)
    out_r = torch.empty_like(out_n)
    lse_r = torch.empty_like(lse_n)
    kernel_out(*args, out_r, lse_r, num_splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(out_n, out_r) and torch.equal(lse_n, lse_r)


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


def test_noalloc_split_reduction_rule():
    """The automatic count an over-large no-alloc call falls back to (host
    arithmetic only, no device call)."""
    lib = _lib.load()
    assert _noalloc_splits(64, 16, 2048) == 0            # 4 splits, 8.7 MB: fits
    assert _noalloc_splits(64, 128, 2048) == 1           # 2 splits need 34.6 MB
    assert _noalloc_splits(96, 128, 2048) == 1
    assert _noalloc_splits(128, 64, 2048) == 1
    # the largest count below the automatic one whose workspace fits
    s = _noalloc_splits(4, 128, 2048)
    assert s == 0 or lib.dsa_attn_workspace_bytes(4, 128, 2048, s) <= _lib.NOALLOC_SCRATCH_BYTES


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
