"""Recorded-workload replay helpers (dsa_amd.trace): loading a safetensors
index file the way the reference driver does (test_splitk_correctness.py:6-18)
and building its inputs.  CPU tests, except the last one (GPU replay)."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle
from conftest import LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, mismatches
from dsa_amd import trace


def _indices(T=1, K=2048, slots=8462 * 64, pad=48, seed=5):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(slots, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    if pad:
        idx[-1, K - pad:] = -1
    return idx


def test_load_sparse_indices_round_trip(tmp_path):
    idx = _indices(T=2)
    p = str(tmp_path / "w.safetensors")
    save_file({"sparse_indices": idx}, p)
    got = trace.load_sparse_indices(p)
    assert got.dtype == torch.int32 and torch.equal(got, idx)
    save_file({"sparse_indices": idx.to(torch.int64)}, p)
    assert torch.equal(trace.load_sparse_indices(p), idx)


def test_load_sparse_indices_rejects_bad_files(tmp_path):
    p = str(tmp_path / "w.safetensors")
    save_file({"other": _indices()}, p)
    with pytest.raises(KeyError):
        trace.load_sparse_indices(p)
    save_file({"sparse_indices": torch.zeros(2048, dtype=torch.int32)}, p)
    with pytest.raises(ValueError):
        trace.load_sparse_indices(p)
    save_file({"sparse_indices": torch.zeros(1, 2048, dtype=torch.float32)}, p)
    with pytest.raises(ValueError):
        trace.load_sparse_indices(p)


def test_workload_inputs_shapes_seed_and_range():
    idx = _indices(slots=256 * 64)
    a = trace.workload_inputs(idx, num_pages=256, seed=3)
    b = trace.workload_inputs(idx, num_pages=256, seed=3)
    assert a["q_nope"].shape == (1, 16, 512) and a["q_pe"].shape == (1, 16, 64)
    assert a["ckv_cache"].shape == (256, 64, 512) and a["kpe_cache"].shape == (256, 64, 64)
    assert a["q_nope"].dtype == torch.bfloat16 and a["sparse_indices"].dtype == torch.int32
    assert torch.equal(a["ckv_cache"], b["ckv_cache"]) and torch.equal(a["q_pe"], b["q_pe"])
    assert abs(a["sm_scale"] - 1.0 / np.sqrt(192.0)) < 1e-12
    with pytest.raises(ValueError):
        trace.workload_inputs(idx, num_pages=100)


@pytest.mark.gpu
def test_replay_matches_splitk_and_oracle(tmp_path):
    """The reference driver's comparison (kernel against kernel_splitk at 4,
    8 and 16 splits) on a synthetic recorded file, plus oracle parity."""
    idx = _indices()
    p = str(tmp_path / "w.safetensors")
    save_file({"sparse_indices": idx}, p)
    errs = trace.replay(p, num_pages=8462, sm_scale=0.1352337788608801, seed=7)
    print("replay errors", errs, flush=True)
    assert max(v for k, v in errs.items() if k.endswith("_out")) <= 1e-2
    assert max(v for k, v in errs.items() if k.endswith("_lse")) <= 1e-3
    d = trace.workload_inputs(idx, num_pages=8462, sm_scale=0.1352337788608801, seed=7)
    from dsa_amd import kernel, workloads
    g = workloads.to_device(d, "cuda:0")
    out, lse = kernel(g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], g["sparse_indices"],
                      d["sm_scale"])
    torch.cuda.synchronize()

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    ref_out, ref_lse = oracle.attention(bits(d["q_nope"]), bits(d["q_pe"]), bits(d["ckv_cache"]),
                                        bits(d["kpe_cache"]), d["sparse_indices"].numpy(),
                                        d["sm_scale"])
    assert mismatches(out.float().cpu().numpy(), oracle.bf16_bits_to_f32(ref_out), OUT_ATOL,
                      OUT_RTOL) == 0
    assert mismatches(lse.cpu().numpy(), ref_lse, LSE_ATOL, LSE_RTOL) == 0
