"""GPU parity of the lightning indexer + top-k and of the indexer -> attention
pipeline, against the CPU oracle.

Scores must match the oracle bit for bit (the exact rounding order of
include/dsa_abi.h) and the selected positions must be the same sets, ties
going to the lower position.  Reference: solution/triton/indexer_kernel.py
:4-343 (score structure :185-275, intended selection :289-343) and the
BASELINE indexer workload (config 5).
"""
import os

import numpy as np
import pytest
import torch

import oracle
from conftest import LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, fill_lds_with_nan, mismatches
from dsa_amd import _lib, workloads
from dsa_amd.indexer_kernel import run_indexer_and_topk, run_sparse_attention_pipeline

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NTHREADS = min(16, os.cpu_count() or 1)


def _np(d):
    return {k: (v.numpy() if isinstance(v, torch.Tensor) and v.dtype != torch.bfloat16 else v)
            for k, v in d.items()}


def _gpu_indexer(d, topk, block_table=None, page_size=64, nan_lds=False):
    g = workloads.to_device(d, DEV)
    bt = None if block_table is None else block_table.to(DEV)
    if nan_lds:
        fill_lds_with_nan(DEV)
    out, scores = run_indexer_and_topk(g["q_idx"], g["k_idx"], g["k_scale"], g["weights"],
                                       g["causal_limit"], topk, block_table=bt,
                                       page_size=page_size, return_scores=True)
    torch.cuda.synchronize()
    return out.cpu().numpy(), scores.cpu().numpy()


def _oracle(d, topk):
    n = _np(d)
    sc = oracle.indexer_scores(n["q_idx"], n["k_idx"], n["k_scale"], n["weights"],
                               n["causal_limit"].astype(np.int64), NTHREADS)
    return oracle.topk(sc, n["causal_limit"].astype(np.int64), topk), sc


def _assert_same(got_idx, got_sc, ref_idx, ref_sc, label):
    bad = np.flatnonzero(got_sc.view(np.uint32) != ref_sc.view(np.uint32))
    assert bad.size == 0, (f"{label}: {bad.size} scores differ from the oracle, first at "
                           f"{np.unravel_index(bad[0], ref_sc.shape)}: {got_sc.flat[bad[0]]!r} vs "
                           f"{ref_sc.flat[bad[0]]!r}")
    for t in range(ref_idx.shape[0]):
        assert np.array_equal(np.sort(got_idx[t]), np.sort(ref_idx[t])), f"{label}: row {t} set differs"
        valid = got_idx[t][got_idx[t] >= 0]
        assert np.all(np.diff(valid) > 0), f"{label}: row {t} not in ascending position order"


def test_cfg5_indexer_full_bit_exact():
    d = workloads.indexer_inputs(seed=workloads.DEFAULT_SEED + 5)
    got_idx, got_sc = _gpu_indexer(d, 2048)
    ref_idx, ref_sc = _oracle(d, 2048)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, "cfg5")


@pytest.mark.parametrize("T,Hi,S,topk", [(5, 16, 1000, 64), (3, 32, 777, 300), (33, 48, 513, 17),
                                         (2, 64, 300, 512)])
def test_ragged_shapes(T, Hi, S, topk):
    d = workloads.indexer_inputs(T=T, Hi=Hi, S=S, seed=T * 1000 + S)
    got_idx, got_sc = _gpu_indexer(d, topk)
    ref_idx, ref_sc = _oracle(d, topk)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, f"T={T} Hi={Hi} S={S} k={topk}")


@pytest.mark.parametrize("T,Hi,S", [(22, 32, 3000), (5, 48, 2203), (9, 64, 4099), (1, 64, 900)])
def test_chunked_ranges_random_causal_limits(T, Hi, S):
    """Causal limits anywhere in a token's row.  The three-product path deals
    a range out in chunks of six blocks to the token's two waves; a limit
    cuts the last chunk after 1..6 blocks (with these shapes every remainder
    occurs), masks part of its last block and leaves later blocks at -inf.
    T not a multiple of 4 leaves workgroups with fewer tokens."""
    d = workloads.indexer_inputs(T=T, Hi=Hi, S=S, seed=T * 7919 + S)
    lim = np.random.default_rng(S).integers(-3, S, T)
    d["causal_limit"] = torch.from_numpy(lim.astype(np.int32))
    topk = min(256, S // 2)
    got_idx, got_sc = _gpu_indexer(d, topk)
    ref_idx, ref_sc = _oracle(d, topk)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, f"T={T} Hi={Hi} S={S}")


@pytest.mark.parametrize("scale,label", [(60.0, "third piece"), (28.0, "beyond the int32 combine")])
def test_one_wide_block_sends_its_range_to_the_general_paths(scale, label):
    """One block of 16 positions with large values: the position range that
    holds it takes the general paths (split between the token's two waves),
    every other range the three-product path."""
    T, Hi, S = 6, 64, 5000
    d = workloads.indexer_inputs(T=T, Hi=Hi, S=S, seed=99)
    g = torch.Generator().manual_seed(99)
    k = d["k_idx"].view(torch.float8_e4m3fn).float()
    k[592:608] = (torch.randn(16, 128, generator=g) * scale).clamp(-scale, scale)
    d["k_idx"] = workloads.e4m3(k)
    got_idx, got_sc = _gpu_indexer(d, 300)
    ref_idx, ref_sc = _oracle(d, 300)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, label)


def test_ties_go_to_lower_positions():
    d = workloads.indexer_inputs(T=4, Hi=16, S=600, seed=7)
    k = d["k_idx"].clone()
    k[300:600] = k[0:300]                      # exact duplicate rows ...
    sc = d["k_scale"].clone()
    sc[300:600] = sc[0:300]                    # ... with the same scales: tied scores
    d.update(k_idx=k, k_scale=sc)
    for topk in (1, 100, 333, 590):
        got_idx, got_sc = _gpu_indexer(d, topk)
        ref_idx, ref_sc = _oracle(d, topk)
        _assert_same(got_idx, got_sc, ref_idx, ref_sc, f"ties k={topk}")
    d["weights"] = torch.zeros_like(d["weights"])   # every score 0: the first k positions win
    got_idx, _ = _gpu_indexer(d, 50)
    assert np.array_equal(got_idx, np.tile(np.arange(50, dtype=np.int32), (4, 1)))


@pytest.mark.parametrize("n_tied,topk", [(40, 30), (150, 100), (300, 200), (150, 150)])
def test_tied_top_group_every_selection_path(n_tied, topk):
    """The top `n_tied` scores of each row are exactly equal (identical key
    rows) and the k-th largest lies among them: the register top-k then
    ranks up to 64 survivors with ballots, up to 256 pairwise, and more
    takes two further radix passes.  Every path must take the lowest
    positions of the tie."""
    g = torch.Generator().manual_seed(n_tied)
    T, Hi, S = 3, 16, 4096
    q = torch.ones(T, Hi, 128)
    k = torch.randn(S, 128, generator=g)
    k[:n_tied] = 2.0                                   # dot = 256 against ~N(0, 11)
    perm = torch.randperm(S, generator=g)             # spread the tied rows over the row
    k = k[perm]
    d = {"q_idx": workloads.e4m3(q), "k_idx": workloads.e4m3(k),
         "k_scale": torch.ones(S), "weights": torch.full((T, Hi), 1.0 / Hi),
         "causal_limit": torch.tensor([S - 1, S - 7, S - 1000], dtype=torch.int32)}
    got_idx, got_sc = _gpu_indexer(d, topk)
    ref_idx, ref_sc = _oracle(d, topk)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, f"tied group {n_tied}, k={topk}")
    tied_pos = np.sort(np.flatnonzero(np.isin(perm.numpy(), np.arange(n_tied))))
    for t in range(T):
        n = int(d["causal_limit"][t]) + 1
        want = tied_pos[tied_pos < n][:topk]           # the lowest tied positions win
        assert np.isin(want, got_idx[t]).all(), f"row {t}"
        if len(want) == topk:
            assert np.array_equal(got_idx[t], want), f"row {t}"


@pytest.mark.parametrize("topk", [1, 64, 1000])
def test_outlier_scores_crowd_the_linear_bins(topk):
    """A few huge scores stretch the row's score range, so the top-k's
    histogram of 2048 bins linear in the score puts nearly every key in a
    handful of bins and the k-th largest's bin is crowded: the selection
    must fall back to its radix passes and stay exact (rows 0-1); row 2 has
    an ordinary spread."""
    g = torch.Generator().manual_seed(71)
    T, Hi, S = 3, 16, 6000
    q = torch.ones(T, Hi, 128)
    q[2] = torch.randn(Hi, 128, generator=g)
    k = torch.randn(S, 128, generator=g)
    k[[17, 4000, 5999]] = 400.0                        # dot ~ 51200 against ~N(0, 11)
    d = {"q_idx": workloads.e4m3(q), "k_idx": workloads.e4m3(k),
         "k_scale": torch.ones(S), "weights": torch.full((T, Hi), 1.0 / Hi),
         "causal_limit": torch.tensor([S - 1, S - 2, S - 1], dtype=torch.int32)}
    print(f"outlier scores k={topk}", flush=True)
    got_idx, got_sc = _gpu_indexer(d, topk)
    ref_idx, ref_sc = _oracle(d, topk)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, f"outliers k={topk}")


def test_large_values_take_the_wide_paths():
    """|value| >= 32 needs the third 7-bit piece (fp64 combine), and large
    dots overflow the int32 fast combine; both must stay exact."""
    g = torch.Generator().manual_seed(11)
    T, Hi, S = 3, 16, 400
    q = (torch.randn(T, Hi, 128, generator=g) * 40).clamp(-440, 440)
    k = (torch.randn(S, 128, generator=g) * 40).clamp(-440, 440)
    q[0] = 1.0                                   # a token with only small values
    d = {"q_idx": workloads.e4m3(q), "k_idx": workloads.e4m3(k),
         "k_scale": torch.rand(S, generator=g) + 0.5,
         "weights": torch.randn(T, Hi, generator=g),
         "causal_limit": torch.tensor([S - 1, S - 50, 10], dtype=torch.int32)}
    got_idx, got_sc = _gpu_indexer(d, 128)
    ref_idx, ref_sc = _oracle(d, 128)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, "large values")
    # moderate values: no third piece, but products beyond the int32 fast path
    d2 = dict(d, q_idx=workloads.e4m3((q / 2).clamp(-31, 31)), k_idx=workloads.e4m3((k / 2).clamp(-31, 31)))
    got_idx, got_sc = _gpu_indexer(d2, 128)
    ref_idx, ref_sc = _oracle(d2, 128)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, "moderate values")


def test_short_rows_pad_with_minus_one():
    d = workloads.indexer_inputs(T=4, Hi=16, S=256, seed=3)
    d["causal_limit"] = torch.tensor([-1, 0, 9, 255], dtype=torch.int32)
    got_idx, got_sc = _gpu_indexer(d, 20)
    ref_idx, ref_sc = _oracle(d, 20)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, "short rows")
    assert (got_idx[0] == -1).all() and (got_idx[1][1:] == -1).all() and got_idx[1][0] == 0
    assert (got_idx[2][10:] == -1).all()


def test_block_table_maps_positions_to_slots():
    d = workloads.indexer_inputs(T=6, Hi=32, S=1024, seed=5)
    shared = torch.randperm(16, generator=torch.Generator().manual_seed(1)).to(torch.int32)
    per_tok = torch.stack([torch.randperm(16, generator=torch.Generator().manual_seed(t))
                           for t in range(6)]).to(torch.int32)
    ref_idx, _ = _oracle(d, 100)
    for bt in (shared, per_tok):
        got, _ = _gpu_indexer(d, 100, block_table=bt, page_size=64)
        for t in range(6):
            row = bt if bt.dim() == 1 else bt[t]
            want = workloads.positions_to_slots(torch.from_numpy(ref_idx[t]).long(), row, 64).numpy()
            assert np.array_equal(np.sort(got[t]), np.sort(want))


def test_cfg5_pipeline_end_to_end():
    d = workloads.cfg5()
    g = workloads.to_device(d, DEV)
    out, lse, slots = run_sparse_attention_pipeline(
        g["q_idx"], g["k_idx"], g["k_scale"], g["weights"], g["causal_limit"], g["block_table"],
        g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], d["sm_scale"], topk=2048)
    torch.cuda.synchronize()
    ref_pos, _ = _oracle(d, 2048)
    ref_slots = workloads.positions_to_slots(torch.from_numpy(ref_pos).long(), d["block_table"], 64)
    got_slots = slots.cpu()
    for t in range(got_slots.shape[0]):
        assert torch.equal(torch.sort(got_slots[t]).values, torch.sort(ref_slots[t]).values)

    def bits(x):
        return x.contiguous().view(torch.int16).numpy().view(np.uint16)

    ref_out, ref_lse = oracle.attention(bits(d["q_nope"]), bits(d["q_pe"]), bits(d["ckv_cache"]),
                                        bits(d["kpe_cache"]), ref_slots.numpy(), d["sm_scale"],
                                        NTHREADS)
    assert mismatches(out.float().cpu().numpy(), oracle.bf16_bits_to_f32(ref_out), OUT_ATOL, OUT_RTOL) == 0
    assert mismatches(lse.cpu().numpy(), ref_lse, LSE_ATOL, LSE_RTOL) == 0


@pytest.mark.parametrize("T,Hi,S,topk", [(8, 64, 5000, 2048), (33, 48, 513, 17), (2, 16, 50000, 700),
                                         (2, 16, 70000, 700), (3, 64, 9000, 300)])
def test_after_nan_filled_lds(T, Hi, S, topk):
    """Scores and selections (register top-k of 16 and 64 keys per thread,
    the streaming top-k, rows shorter than top-k) right after a kernel that
    left NaN in every CU's LDS: every LDS location the indexer kernels read
    was written by them first, or the scores and sets would differ."""
    d = workloads.indexer_inputs(T=T, Hi=Hi, S=S, seed=9100 + S)
    ref_idx, ref_sc = _oracle(d, topk)
    for r in range(3):
        print(f"NaN-filled LDS indexer T={T} Hi={Hi} S={S} topk={topk} call {r}", flush=True)
        got_idx, got_sc = _gpu_indexer(d, topk, nan_lds=True)
        _assert_same(got_idx, got_sc, ref_idx, ref_sc, f"T={T} S={S} call {r}")


@pytest.mark.parametrize("S", [12000, 50000, 70000])
def test_long_rows_every_topk_variant(S):
    """Rows of 12000 / 50000 positions use the register top-k with 16 / 64
    keys per thread; 70000 positions the streaming top-k."""
    d = workloads.indexer_inputs(T=2, Hi=16, S=S, seed=S)
    d["causal_limit"] = torch.tensor([S - 1, S // 2], dtype=torch.int32)
    got_idx, got_sc = _gpu_indexer(d, 700)
    ref_idx, ref_sc = _oracle(d, 700)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, f"S={S}")


@pytest.mark.parametrize("S", [3000, 40000])
def test_causal_limit_extremes(S):
    """Limits at the ends of int32 (INT32_MAX: no limit; INT32_MIN: no
    candidate), around S and around 0, in the register top-k (S=3000) and the
    streaming one (S=40000), against the oracle (int64 limits)."""
    lims = [2**31 - 1, -2**31, S - 1, S, S - 2, -1, 0, 1]
    d = workloads.indexer_inputs(T=len(lims), Hi=16, S=S, seed=7 + S)
    d["causal_limit"] = torch.tensor(lims, dtype=torch.int32)
    print(f"causal limit extremes S={S}", flush=True)
    got_idx, got_sc = _gpu_indexer(d, 300)
    ref_idx, ref_sc = _oracle(d, 300)
    _assert_same(got_idx, got_sc, ref_idx, ref_sc, f"limit extremes S={S}")
    assert (got_idx[0] >= 0).all() and (got_idx[1] == -1).all()


def test_graph_replays_match_eager():
    d = workloads.indexer_inputs(T=8, Hi=64, S=5000, seed=21)
    g = workloads.to_device(d, DEV)
    args = (g["q_idx"], g["k_idx"], g["k_scale"], g["weights"], g["causal_limit"])
    eager = run_indexer_and_topk(*args, 256).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_indexer_and_topk(*args, 256)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run_indexer_and_topk(*args, 256)
    for _ in range(3):
        out.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        run_indexer_and_topk(*args, 100)   # eager work between replays
        torch.cuda.synchronize()


# ---- paged fp8 K cache ---------------------------------------------------

def _bf16_rows(g, n):
    """bf16 rows with a spread of magnitudes, a zero row, -0.0 and tiny rows."""
    k = torch.randn(n, 128, generator=g) * torch.exp2(torch.randint(-12, 12, (n, 1), generator=g).float())
    k[0] = 0.0
    k[1, 7] = -0.0
    k[2] *= 1e-30                                   # amax below the 1e-4 floor
    k[3, :64] = 3e4                                  # large, many equal magnitudes
    return k.to(torch.bfloat16)


def test_k_append_matches_oracle_bit_exact():
    """Quantise-on-append writes exactly the oracle's codes and fp32 scales to
    each slot's place in the page layout and leaves every other byte alone
    (negative and out-of-range slots are skipped)."""
    from dsa_amd import k_append
    g = torch.Generator().manual_seed(41)
    ps, pages, n = 64, 40, 1500
    k = _bf16_rows(g, n)
    slots = torch.randperm(pages * ps, generator=g)[:n].to(torch.int32)
    slots[10] = -1
    slots[11] = pages * ps + 5
    base = torch.randint(0, 256, (pages, ps * 132), generator=g, dtype=torch.uint8)
    cache = base.to(DEV)
    print("k_append n=1500 pages=40 ps=64", flush=True)
    k_append(k.to(DEV), slots.to(DEV), cache)
    torch.cuda.synchronize()
    codes, scale = oracle.quantize_k(k.float().numpy())
    want = oracle.pack_k_cache(base.numpy(), codes, scale, slots.numpy(), ps)
    got = cache.cpu().numpy()
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} bytes differ, first at {np.unravel_index(bad[0], got.shape)}"
    # strided rows (a view of a wider tensor) give the same bytes
    wide = torch.zeros(n, 256, dtype=torch.bfloat16)
    wide[:, 64:192] = k
    cache2 = base.to(DEV)
    k_append(wide.to(DEV)[:, 64:192], slots.to(DEV), cache2)
    torch.cuda.synchronize()
    assert torch.equal(cache2.cpu(), cache.cpu())


def test_paged_indexer_equals_flat_bit_for_bit():
    """The indexer over a paged K cache (pages in a random order, appended by
    k_append) returns the same scores and slots as the flat call over the
    same codes and scales."""
    from dsa_amd import k_append, new_k_cache, run_indexer_and_topk_paged
    g = torch.Generator().manual_seed(42)
    T, Hi, S, ps, topk = 12, 64, 6000, 64, 512
    d = workloads.indexer_inputs(T=T, Hi=Hi, S=S, seed=43)
    k = torch.randn(S, 128, generator=g).to(torch.bfloat16)
    n_pages = -(-S // ps) + 3
    page_of = torch.randperm(n_pages, generator=g)[:-(-S // ps)].to(torch.int32)  # position page -> cache page
    pos = torch.arange(S)
    slots = (page_of[pos // ps] * ps + pos % ps).to(torch.int32)
    cache = new_k_cache(n_pages, ps, DEV)
    k_append(k.to(DEV), slots.to(DEV), cache)
    codes, scale = oracle.quantize_k(k.float().numpy())
    flat = dict(d, k_idx=torch.from_numpy(codes), k_scale=torch.from_numpy(scale))
    ref_idx, ref_sc = _gpu_indexer(flat, topk)
    gd = workloads.to_device(d, DEV)
    out, sc = run_indexer_and_topk_paged(gd["q_idx"], cache, page_of.to(DEV), S, gd["weights"],
                                         gd["causal_limit"], topk, return_scores=True)
    torch.cuda.synchronize()
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), ref_sc.view(np.uint32))
    assert np.array_equal(out.cpu().numpy(), ref_idx)
    ora_idx, ora_sc = _oracle(flat, topk)
    _assert_same(ref_idx, ref_sc, ora_idx, ora_sc, "flat over the quantised K")


def test_pipeline_over_paged_k_cache_equals_flat():
    """cfg5's indexer K packed into a paged cache that shares the attention's
    block table: the pipeline gives the same slots, output and lse as over the
    flat K."""
    d = workloads.cfg5()
    g = workloads.to_device(d, DEV)
    ps = 64
    S = d["k_idx"].shape[0]
    bt = d["block_table"]
    assert bt.dim() == 1
    pos = torch.arange(S)
    slots = (bt[pos // ps].long() * ps + pos % ps).numpy()
    base = np.zeros((bt.numel(), ps * 132), np.uint8)
    cache = oracle.pack_k_cache(base, d["k_idx"].view(torch.uint8).numpy(), d["k_scale"].numpy(),
                                slots, ps)
    args = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], d["sm_scale"])
    flat = run_sparse_attention_pipeline(g["q_idx"], g["k_idx"], g["k_scale"], g["weights"],
                                         g["causal_limit"], g["block_table"], *args, topk=2048)
    paged = run_sparse_attention_pipeline(g["q_idx"], None, None, g["weights"], g["causal_limit"],
                                          g["block_table"], *args, topk=2048,
                                          k_cache=torch.from_numpy(cache).to(DEV), num_positions=S)
    torch.cuda.synchronize()
    for a, b in zip(flat, paged):
        assert torch.equal(a, b)


def test_paged_indexer_unmapped_pages_read_as_zero_rows():
    """k_pages entries outside [0, pages) (a -1 or a stale id) read as zero
    codes with scale 0 -- score 0 -- and nothing outside the cache is read:
    the result equals the flat call with those positions zeroed."""
    from dsa_amd import k_append, new_k_cache, run_indexer_and_topk_paged
    g = torch.Generator().manual_seed(52)
    T, Hi, S, ps, topk = 6, 32, 1000, 64, 200
    d = workloads.indexer_inputs(T=T, Hi=Hi, S=S, seed=53)
    n_pages = -(-S // ps)
    k = torch.randn(S, 128, generator=g).to(torch.bfloat16)
    page_of = torch.arange(n_pages, dtype=torch.int32)
    cache = new_k_cache(n_pages, ps, DEV)
    pos = torch.arange(S)
    k_append(k.to(DEV), (page_of[pos // ps] * ps + pos % ps).to(torch.int32).to(DEV), cache)
    page_of[2] = -1
    page_of[5] = n_pages + 3
    page_of[7] = 2**31 - 1
    codes, scale = oracle.quantize_k(k.float().numpy())
    for pg in (2, 5, 7):
        codes[pg * ps:(pg + 1) * ps] = 0
        scale[pg * ps:(pg + 1) * ps] = 0.0
    flat = dict(d, k_idx=torch.from_numpy(codes), k_scale=torch.from_numpy(scale))
    ref_idx, ref_sc = _gpu_indexer(flat, topk)
    gd = workloads.to_device(d, DEV)
    print("paged indexer with unmapped pages", flush=True)
    out, sc = run_indexer_and_topk_paged(gd["q_idx"], cache, page_of.to(DEV), S, gd["weights"],
                                         gd["causal_limit"], topk, return_scores=True)
    torch.cuda.synchronize()
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), ref_sc.view(np.uint32))
    assert np.array_equal(out.cpu().numpy(), ref_idx)
    ora_idx, ora_sc = _oracle(flat, topk)
    _assert_same(ref_idx, ref_sc, ora_idx, ora_sc, "flat with zeroed pages")


# ---- prepared K planes ---------------------------------------------------

def test_prepared_planes_give_the_same_bits():
    """Calls reading planes from prepare_k (capacity above the sequence
    length, the K tensors not passed) return the scores and sets of calls
    that prepare K themselves, and those match the oracle; one planes object
    serves several calls."""
    from dsa_amd import prepare_k
    d = workloads.cfg5()
    g = workloads.to_device(d, DEV)
    print("prepared planes cfg5", flush=True)
    planes = prepare_k(g["k_idx"], g["k_scale"], capacity=40000)
    assert planes.num_positions == d["k_idx"].shape[0]
    args = (g["q_idx"], g["k_idx"], g["k_scale"], g["weights"], g["causal_limit"])
    ref, ref_sc = run_indexer_and_topk(*args, 2048, return_scores=True)
    for topk in (2048, 77):
        out, sc = run_indexer_and_topk(g["q_idx"], None, None, g["weights"], g["causal_limit"],
                                       topk, return_scores=True, k_planes=planes)
        torch.cuda.synchronize()
        assert torch.equal(sc.view(torch.int32), ref_sc.view(torch.int32))
        if topk == 2048:
            assert torch.equal(out, ref)
    ora_idx, ora_sc = _oracle(d, 2048)
    _assert_same(ref.cpu().numpy(), ref_sc.cpu().numpy(), ora_idx, ora_sc, "cfg5 with planes")
    # the pipeline with planes gives the same slots, output and lse
    a = (g["q_nope"], g["q_pe"], g["ckv_cache"], g["kpe_cache"], d["sm_scale"])
    p1 = run_sparse_attention_pipeline(*args, g["block_table"], *a, topk=2048)
    p2 = run_sparse_attention_pipeline(g["q_idx"], None, None, g["weights"], g["causal_limit"],
                                       g["block_table"], *a, topk=2048, k_planes=planes)
    torch.cuda.synchronize()
    for x, y in zip(p1, p2):
        assert torch.equal(x, y)


def test_planes_refreshed_after_appends_match_a_full_preparation():
    """A paged K cache grows by appends of uneven lengths (some ending inside
    a 16-position block); after each append only the appended positions are
    re-prepared.  The planes then equal a full preparation byte for byte and
    the indexer over them equals the paged call without planes."""
    from dsa_amd import KPlanes, k_append, new_k_cache, prepare_k_paged, run_indexer_and_topk_paged
    gen = torch.Generator().manual_seed(61)
    T, Hi, ps, topk = 8, 64, 64, 300
    S_max = 3000
    n_pages = -(-S_max // ps) + 2
    page_of = torch.randperm(n_pages, generator=gen).to(torch.int32)
    k = torch.randn(S_max, 128, generator=gen).to(torch.bfloat16)
    pos = torch.arange(S_max)
    slots = (page_of[pos // ps].long() * ps + pos % ps).to(torch.int32)
    cache = new_k_cache(n_pages, ps, DEV)
    pages = page_of.to(DEV)
    planes = KPlanes(S_max, DEV)
    S = 0
    for n in (1000, 7, 9, 16, 1, 500, 1467):
        k_append(k[S:S + n].to(DEV), slots[S:S + n].to(DEV), cache)
        print(f"append {n} at {S}", flush=True)
        prepare_k_paged(cache, pages, S + n, planes=planes, first_position=S)
        S += n
        full = prepare_k_paged(cache, pages, S, capacity=S_max)
        torch.cuda.synchronize()
        # blocks past S hold whatever earlier refreshes left; compare the
        # regions the indexer reads for S positions
        nkb = (S + 15) // 16
        kpb = nkb * 6144
        kmax_off = (((S_max + 15) // 16) * 6144 + 255) // 256 * 256
        cs_off = kmax_off + ((((S_max + 15) // 16) * 4 + 255) // 256 * 256)
        for lo, hi in ((0, kpb), (kmax_off, kmax_off + nkb * 4), (cs_off, cs_off + S * 4)):
            assert torch.equal(planes.buf[lo:hi], full.buf[lo:hi]), (S, lo)
        assert _lib.load().dsa_indexer_k_planes_bytes(S_max) == planes.buf.numel()
        d = workloads.indexer_inputs(T=T, Hi=Hi, S=S, seed=62 + S)
        gd = workloads.to_device(d, DEV)
        ref, ref_sc = run_indexer_and_topk_paged(gd["q_idx"], cache, pages, S, gd["weights"],
                                                 gd["causal_limit"], topk, return_scores=True)
        out, sc = run_indexer_and_topk(gd["q_idx"], None, None, gd["weights"], gd["causal_limit"],
                                       topk, return_scores=True, k_planes=planes)
        torch.cuda.synchronize()
        assert torch.equal(sc.view(torch.int32), ref_sc.view(torch.int32)), S
        assert torch.equal(out, ref), S


def test_planes_in_graph_replays_match_eager():
    from dsa_amd import prepare_k
    d = workloads.indexer_inputs(T=8, Hi=64, S=5000, seed=63)
    g = workloads.to_device(d, DEV)
    planes = prepare_k(g["k_idx"], g["k_scale"])
    args = (g["q_idx"], None, None, g["weights"], g["causal_limit"])
    eager = run_indexer_and_topk(*args, 256, k_planes=planes).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_indexer_and_topk(*args, 256, k_planes=planes)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run_indexer_and_topk(*args, 256, k_planes=planes)
    for _ in range(3):
        out.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
