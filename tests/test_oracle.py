"""Pins the CPU oracle (CPU only, no GPU).

The reference commits no golden vectors for this path, and its own checker,
run() in solution/triton/indexer_kernel.py:436-497, cannot run as written
(`math` is never imported).  The oracle is therefore pinned by:

* library routines: torch's bf16 and e4m3fn casts, torch's float64
  scaled_dot_product_attention and logsumexp, numpy's lexsort;
* closed forms: one valid slot, q = 0, all-padding rows, duplicate slots;
* invariances: permutation of a row, -1 anywhere == deletion, page-size
  views, a constant logit shift through the kpe term;
* an independent exact integer computation of the indexer scores.

Each check is chosen so a plausible slip (dropped q_pe.kpe term, natural-log
lse, missing normalisation, transposed operand, wrong tie order) fails it.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

LN2 = math.log(2.0)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _rand_case(T, H, K, slots, ps, seed, pad_frac=0.0, var=0.5):
    g = torch.Generator().manual_seed(seed)
    qn = torch.randn(T, H, 512, generator=g).to(torch.bfloat16)
    qp = torch.randn(T, H, 64, generator=g).to(torch.bfloat16)
    ckv = (torch.randn(slots // ps, ps, 512, generator=g) * math.sqrt(var)).to(torch.bfloat16)
    kpe = (torch.randn(slots // ps, ps, 64, generator=g) * math.sqrt(var)).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(slots, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    if pad_frac:
        m = torch.rand(T, K, generator=g) < pad_frac
        idx[m] = -1
    return qn, qp, ckv, kpe, idx


def _oracle(qn, qp, ckv, kpe, idx, scale):
    return oracle.attention(_bits(qn), _bits(qp), _bits(ckv), _bits(kpe), idx.numpy(), scale)


def _sdpa_reference(qn, qp, ckv, kpe, idx, scale):
    """torch float64 scaled_dot_product_attention + logsumexp per token."""
    T, H, _ = qn.shape
    kc_all = ckv.reshape(-1, 512).double()
    kp_all = kpe.reshape(-1, 64).double()
    out = torch.zeros(T, H, 512, dtype=torch.float64)
    lse = torch.full((T, H), -math.inf, dtype=torch.float64)
    for t in range(T):
        sel = idx[t][idx[t] >= 0].long()
        if sel.numel() == 0:
            continue
        q = torch.cat([qn[t].double(), qp[t].double()], -1)[None]          # [1,H,576]
        k = torch.cat([kc_all[sel], kp_all[sel]], -1)[None, None].expand(1, H, -1, -1)
        v = kc_all[sel][None, None].expand(1, H, -1, -1)
        out[t] = F.scaled_dot_product_attention(q[:, :, None, :], k, v, scale=scale)[0, :, 0]
        lse[t] = torch.logsumexp((q[0] @ k[0, 0].T) * scale, dim=-1) / LN2
    return out, lse


def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(1)
    x = torch.cat([torch.randn(100000, generator=g) * 10 ** torch.randint(-30, 30, (100000,), generator=g),
                   torch.tensor([0.0, -0.0, 1.0, -1.0, 3.0e38, -3.0e38, float("inf"), -float("inf"),
                                 1.00390625, 1.01171875, 1.0 + 2 ** -9, 1.0 + 3 * 2 ** -9])])
    want = _bits(x.to(torch.bfloat16))
    got = oracle.f32_to_bf16_bits(x.numpy())
    assert np.array_equal(got, want)
    lib = oracle._load()
    for v in x[-12:].tolist() + x[:2000].tolist():
        assert lib.oracle_f32_to_bf16(v) == _bits(torch.tensor([v]).to(torch.bfloat16))[0]


def test_e4m3_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.e4m3_decode(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and nan.sum() == 2
    assert np.array_equal(got[~nan], want[~nan])


@pytest.mark.parametrize("T,H,K,slots,ps,pad", [(3, 16, 40, 256, 1, 0.0), (4, 32, 64, 512, 4, 0.3),
                                                (2, 16, 7, 64, 64, 0.5)])
def test_attention_matches_torch_sdpa(T, H, K, slots, ps, pad):
    scale = 1 / math.sqrt(192)
    qn, qp, ckv, kpe, idx = _rand_case(T, H, K, slots, ps, seed=T * 100 + K, pad_frac=pad)
    out_bits, lse = _oracle(qn, qp, ckv, kpe, idx, scale)
    ref_out, ref_lse = _sdpa_reference(qn, qp, ckv, kpe, idx, scale)
    got = oracle.bf16_bits_to_f32(out_bits).astype(np.float64)
    want = ref_out.numpy()
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want) <= ulp)
    assert np.allclose(lse, ref_lse.numpy(), rtol=1e-6, atol=1e-6)


def test_single_slot_closed_form():
    qn, qp, ckv, kpe, _ = _rand_case(2, 16, 1, 128, 1, seed=7)
    idx = torch.tensor([[5, -1, -1], [-1, 77, -1]], dtype=torch.int32)
    out_bits, lse = _oracle(qn, qp, ckv, kpe, idx, 0.3)
    for t, s in ((0, 5), (1, 77)):
        assert np.array_equal(out_bits[t], np.tile(_bits(ckv.reshape(-1, 512)[s]), (16, 1)))
        logit = (qn[t].double() @ ckv.reshape(-1, 512)[s].double()
                 + qp[t].double() @ kpe.reshape(-1, 64)[s].double()) * 0.3
        assert np.allclose(lse[t], (logit / LN2).numpy(), rtol=1e-6, atol=1e-6)


def test_zero_query_gives_mean_and_log2_count():
    _, _, ckv, kpe, idx = _rand_case(2, 16, 24, 300, 3, seed=9)
    qn = torch.zeros(2, 16, 512, dtype=torch.bfloat16)
    qp = torch.zeros(2, 16, 64, dtype=torch.bfloat16)
    idx[1, ::3] = -1
    out_bits, lse = _oracle(qn, qp, ckv, kpe, idx, 0.125)
    for t in range(2):
        sel = idx[t][idx[t] >= 0].long()
        mean = ckv.reshape(-1, 512)[sel].double().mean(0).float()
        assert np.array_equal(out_bits[t], np.tile(_bits(mean.to(torch.bfloat16)), (16, 1)))
        assert np.allclose(lse[t], math.log2(sel.numel()), atol=1e-6)


def test_empty_rows_and_padding_anywhere():
    qn, qp, ckv, kpe, idx = _rand_case(3, 16, 32, 256, 1, seed=11)
    idx[0] = -1
    padded = idx.clone()
    padded[1, [0, 5, 31]] = -1
    out_a, lse_a = _oracle(qn, qp, ckv, kpe, padded, 0.1)
    assert not out_a[0].any() and np.all(np.isneginf(lse_a[0]))
    # -1 at any position is the same as deleting the entry
    kept = padded[1][padded[1] >= 0][None]
    out_b, lse_b = _oracle(qn[1:2], qp[1:2], ckv, kpe, kept, 0.1)
    assert np.array_equal(out_a[1], out_b[0]) and np.allclose(lse_a[1], lse_b[0], rtol=1e-7)


def test_permutation_and_page_size_invariance():
    qn, qp, ckv, kpe, idx = _rand_case(2, 16, 50, 512, 8, seed=13, pad_frac=0.2)
    out_a, lse_a = _oracle(qn, qp, ckv, kpe, idx, 0.07)
    perm = idx[:, torch.randperm(50, generator=torch.Generator().manual_seed(3))]
    out_b, lse_b = _oracle(qn, qp, ckv, kpe, perm, 0.07)
    flat = _oracle(qn, qp, ckv.reshape(512, 1, 512), kpe.reshape(512, 1, 64), idx, 0.07)
    # fp64 accumulation in a different order: results agree to rounding
    diff = np.abs(oracle.bf16_bits_to_f32(out_a) - oracle.bf16_bits_to_f32(out_b))
    assert diff.max() <= 2 ** -7 * np.abs(oracle.bf16_bits_to_f32(out_a)).max()
    assert np.allclose(lse_a, lse_b, rtol=1e-7)
    assert np.array_equal(out_a, flat[0]) and np.array_equal(lse_a, flat[1])


def test_constant_shift_through_kpe_moves_lse_only():
    qn, qp, ckv, kpe, idx = _rand_case(1, 16, 30, 128, 1, seed=17)
    kpe_const = kpe.clone()
    kpe_const[:] = kpe[0, 0]
    out_a, lse_a = _oracle(qn, qp, ckv, kpe_const, idx, 0.2)
    qp2 = (qp.float() * 2).to(torch.bfloat16)  # doubles the constant q_pe.kpe term
    out_b, lse_b = _oracle(qn, qp2, ckv, kpe_const, idx, 0.2)
    shift = (qp[0].double() @ kpe[0, 0].double()) * 0.2 / LN2  # per head
    assert np.array_equal(out_a, out_b)
    assert np.allclose(lse_b[0] - lse_a[0], shift.numpy(), atol=1e-5)


def test_duplicate_slots_count_twice():
    qn, qp, ckv, kpe, _ = _rand_case(1, 16, 1, 64, 1, seed=19)
    one = torch.tensor([[3]], dtype=torch.int32)
    two = torch.tensor([[3, 3]], dtype=torch.int32)
    o1, l1 = _oracle(qn, qp, ckv, kpe, one, 0.1)
    o2, l2 = _oracle(qn, qp, ckv, kpe, two, 0.1)
    assert np.array_equal(o1, o2) and np.allclose(l2, l1 + 1.0, atol=1e-6)


def test_out_of_range_slot_raises():
    qn, qp, ckv, kpe, idx = _rand_case(1, 16, 4, 64, 1, seed=23)
    idx[0, 2] = 64
    with pytest.raises(ValueError):
        _oracle(qn, qp, ckv, kpe, idx, 0.1)


# ---------------------------------------------------------------- indexer

def _f32_nearest_even(x: Fraction) -> np.float32:
    """Exact rational -> nearest float32, ties to even (finite range)."""
    f = np.float32(float(x))                      # within one ulp of the answer
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = None
    for c in cands:
        d = abs(Fraction(float(c)) - x)
        even = (int(np.array(c, np.float32).view(np.uint32)) & 1) == 0
        if best is None or d < best[0] or (d == best[0] and even):
            best = (d, c)
    return np.float32(best[1])


def _fma32(a, b, c) -> np.float32:
    return _f32_nearest_even(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _exact_scores_independent(q, k, scale, w, limit):
    """Independent restatement: integer dot products (values x 2^9 are
    integers for every finite e4m3 code), then the documented fp32 rounding
    sequence: exact-rational fma per head within four head groups, pairwise
    group sum, then the scale."""
    tab = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).double()
    tab = torch.nan_to_num(tab, nan=0.0).numpy()
    qi = np.round(tab[q] * 512).astype(np.int64)     # [T,Hi,D]
    ki = np.round(tab[k] * 512).astype(np.int64)     # [S,D]
    T, Hi, _ = q.shape
    S = k.shape[0]
    dots = np.einsum("thd,sd->tsh", qi, ki)          # exact int64, = d * 2^18
    out = np.empty((T, S), np.float32)
    f = np.float32
    quarter = Hi // 4
    for t in range(T):
        for s in range(S):
            if s > limit[t]:
                out[t, s] = -np.inf
                continue
            G = []
            for gi in range(4):
                acc = f(0.0)
                for h in range(gi * quarter, (gi + 1) * quarter):
                    r = f(float(max(int(dots[t, s, h]), 0)))   # int -> fp32, one rounding
                    acc = _fma32(w[t, h], r, acc)
                G.append(acc)
            total = f(f(G[0] + G[1]) + f(G[2] + G[3]))
            out[t, s] = f(total * f(f(scale[s]) * f(2.0 ** -18)))
    return out, dots


def test_fma32_helper_rounds_exactly():
    # 1 + 2^-24 is a tie between 1 and 1 + 2^-23: to even (1.0); a fused
    # product keeps the bits a separate multiply would drop
    assert _f32_nearest_even(Fraction(1) + Fraction(1, 2 ** 24)) == np.float32(1.0)
    assert _f32_nearest_even(Fraction(1) + Fraction(3, 2 ** 24)) == np.float32(1.0 + 2.0 ** -22)
    a = np.float32(1.0 + 2.0 ** -12)
    fused = _fma32(a, a, np.float32(-1.0))
    assert fused == np.float32(2.0 ** -11 + 2.0 ** -24)
    assert np.float32(np.float32(a * a) - np.float32(1.0)) != fused


def _indexer_case(T, Hi, S, seed, dup_rows=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, Hi, 128, generator=g).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    kf = torch.randn(S, 128, generator=g)
    if dup_rows:
        kf[S - dup_rows:] = kf[:dup_rows]
    k = kf.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    scale = (torch.rand(S, generator=g) * 1.5 + 0.5).numpy()
    if dup_rows:
        scale[S - dup_rows:] = scale[:dup_rows]
    w = (torch.randn(T, Hi, generator=g) / math.sqrt(8)).numpy()
    limit = np.array([S - T + t for t in range(T)], np.int64)
    return q, k, scale, w, limit


def test_indexer_scores_bit_exact_vs_integer_restatement():
    q, k, scale, w, limit = _indexer_case(3, 32, 70, seed=5)
    got = oracle.indexer_scores(q, k, scale, w, limit)
    want, dots = _exact_scores_independent(q, k, scale, w, limit)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # and the value is the real-number score up to fp32 rounding
    tab = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).double().numpy()
    real = (np.maximum((dots * 2.0 ** -18) * scale[None, :, None], 0) * w[:, None, :]).sum(-1)
    mask = np.isfinite(got)
    assert np.allclose(got[mask], real[mask], rtol=1e-5, atol=1e-4)
    assert np.all(np.isneginf(got[~mask])) and (~mask).sum() == sum(70 - 1 - l for l in limit)
    del tab


def test_indexer_zero_weights_and_negative_dots():
    q, k, scale, w, limit = _indexer_case(2, 16, 40, seed=6)
    w[:] = 0.0
    assert np.all(oracle.indexer_scores(q, k, scale, w, limit)[np.isfinite(
        oracle.indexer_scores(q, k, scale, w, limit))] == 0.0)
    w[:] = 1.0
    qneg = q.copy()
    qneg[...] = 0xB8  # e4m3 -1.0
    kpos = k.copy()
    kpos[...] = 0x38  # +1.0: every dot is -128 -> relu gives 0
    sc = oracle.indexer_scores(qneg, kpos, scale, w, limit)
    assert np.all(sc[np.isfinite(sc)] == 0.0)


def test_topk_matches_lexsort_and_ties_go_to_lower_position():
    q, k, scale, w, limit = _indexer_case(4, 16, 300, seed=8, dup_rows=40)
    sc = oracle.indexer_scores(q, k, scale, w, limit)
    K = 64
    got = oracle.topk(sc, limit, K)
    for t in range(4):
        n = int(limit[t]) + 1
        order = np.lexsort((np.arange(n), -sc[t, :n].astype(np.float64)))
        assert np.array_equal(got[t], order[:K])
    # duplicated rows produce exact ties (where both positions are candidates)
    cand = [s for s in range(40) if 300 - 40 + s <= limit[0]]
    assert all(sc[0, s] == sc[0, 300 - 40 + s] for s in cand) and len(cand) == 37
    # all-equal scores: the k lowest positions win
    w0 = np.zeros_like(w)
    flat = oracle.indexer_scores(q, k, scale, w0, limit)
    assert np.array_equal(oracle.topk(flat, limit, K), np.tile(np.arange(K), (4, 1)))


def test_topk_pads_short_rows():
    sc = np.array([[3.0, 1.0, 2.0, 5.0]], np.float32)
    got = oracle.topk(sc, np.array([2]), 5)
    assert got.tolist() == [[0, 2, 1, -1, -1]]


# ---- quantise-on-append into the paged fp8 K cache ----------------------

def test_e4m3_encode_matches_torch_cast_including_ties():
    rng = np.random.default_rng(0)
    vals = oracle.e4m3_decode(np.arange(0x7f))
    mids = (vals[:-1] + vals[1:]) / 2                 # every tie between neighbours
    y = np.concatenate([rng.uniform(-448, 448, 20000), rng.uniform(-0.02, 0.02, 20000), vals,
                        -vals, mids, -mids,
                        [0.0, -0.0, 448.0, -448.0, 2.0 ** -10, 3 * 2.0 ** -11]]).astype(np.float32)
    want = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.e4m3_encode(y), want)


def test_quantize_k_closed_forms():
    rng = np.random.default_rng(1)
    k = rng.standard_normal((6, 128)).astype(np.float32)
    k[1] = 0.0                                         # zero row: floor scale, zero codes
    k[2, 5] = -0.0
    k[3] *= 1e-7                                       # amax below the 1e-4 floor
    codes, scale = oracle.quantize_k(k)
    assert scale.dtype == np.float32 and codes.dtype == np.uint8
    assert scale[1] == np.float32(np.float32(1e-4) / np.float32(448.0)) and not codes[1].any()
    for r in (0, 2, 4, 5):                             # the largest magnitude encodes to +-448
        j = int(np.argmax(np.abs(k[r])))
        assert codes[r, j] == (0xfe if k[r, j] < 0 else 0x7e)
    assert np.abs(oracle.e4m3_decode(codes[3])).max() < 448.0
    # scaling a row by a power of two scales its scale exactly and keeps its codes
    c2, s2 = oracle.quantize_k(k[[0, 4]] * np.float32(64.0))
    assert np.array_equal(c2, codes[[0, 4]]) and np.array_equal(s2, scale[[0, 4]] * np.float32(64.0))
    # decoded values are within half an e4m3 step (relative 2^-4) of k / scale
    dec = oracle.e4m3_decode(codes) * scale[:, None]
    err = np.abs(dec - k)
    assert np.all(err <= np.abs(k) * 2.0 ** -4 + scale[:, None] * 2.0 ** -10 + 1e-30)


def test_k_cache_pack_unpack_roundtrip():
    rng = np.random.default_rng(2)
    ps, pages = 8, 5
    codes = rng.integers(0, 256, (12, 128), dtype=np.uint8)
    scale = rng.uniform(0.001, 2, 12).astype(np.float32)
    slots = rng.permutation(ps * pages)[:12]
    slots[3] = -1                                       # skipped
    base = rng.integers(0, 256, (pages, ps * 132), dtype=np.uint8)
    cache = oracle.pack_k_cache(base, codes, scale, slots, ps)
    keep = slots >= 0
    c, s = oracle.unpack_k_cache(cache, ps, slots[keep])
    assert np.array_equal(c, codes[keep]) and np.array_equal(s, scale[keep])
    touched = np.zeros_like(base, dtype=bool)
    for sl in slots[keep]:
        pg, off = divmod(int(sl), ps)
        touched[pg, off * 128:(off + 1) * 128] = True
        touched[pg, ps * 128 + off * 4:ps * 128 + off * 4 + 4] = True
    assert np.array_equal(cache[~touched], base[~touched])


def test_mismatch_helper_counts_signs_of_infinity_and_nans():
    """The tolerance check of every parity test: fail iff |d| > atol and
    |d| > rtol*|e|; infinities must match in sign, NaN only NaN."""
    from conftest import mismatches
    inf = np.inf
    assert mismatches([inf, -inf], [-inf, inf], 1e-3, 1e-3) == 2
    assert mismatches([inf, -inf], [inf, -inf], 1e-3, 1e-3) == 0
    assert mismatches([-inf, 1.0], [0.0, -inf], 1e-3, 1e-3) == 2
    assert mismatches([np.nan, 1.0], [1.0, np.nan], 1e-3, 1e-3) == 2
    assert mismatches([np.nan], [np.nan], 1e-3, 1e-3) == 0
    # both bounds must be exceeded
    assert mismatches([1.02], [1.0], 1e-2, 1e-2) == 1
    assert mismatches([1.005], [1.0], 1e-2, 1e-2) == 0
    assert mismatches([100.5], [100.0], 1e-2, 1e-2) == 0     # rel 0.5 % passes
    assert mismatches([0.015], [0.0], 1e-2, 1e-2) == 1


def test_torch_fp32_restatement_matches_fp64_oracle():
    """oracle.torch_ref.run_fp32 (the CPU baseline bench.py times) agrees with
    the pinned fp64 oracle within the reference checker's tolerances, on
    padded, empty, duplicate-slot and outlier rows and several page sizes."""
    from conftest import LSE_ATOL, LSE_RTOL, OUT_ATOL, OUT_RTOL, mismatches
    from oracle.torch_ref import run_fp32
    for T, H, K, slots, ps, pad in ((4, 16, 256, 4096, 1, 0.2), (3, 32, 100, 1024, 64, 0.0),
                                    (2, 48, 33, 128, 4, 0.5)):
        qn, qp, ckv, kpe, idx = _rand_case(T, H, K, slots, ps, seed=500 + K, pad_frac=pad)
        ckv.view(-1, 512)[::13] *= 8                      # outlier rows
        idx[0] = -1                                        # an empty row
        idx[-1, 1] = idx[-1, 0]                            # a duplicate slot counts twice
        scale = 1 / math.sqrt(192)
        out, lse = run_fp32(qn, qp, ckv, kpe, idx, scale)
        ref_bits, ref_lse = _oracle(qn, qp, ckv, kpe, idx, scale)
        want = oracle.bf16_bits_to_f32(ref_bits)
        assert mismatches(out.float().numpy(), want, OUT_ATOL, OUT_RTOL) == 0
        assert mismatches(lse.numpy(), ref_lse, LSE_ATOL, LSE_RTOL) == 0
        assert torch.isneginf(lse[0]).all() and not out[0].float().abs().sum()


def _real_scores_and_band(q, k, scale, w, limit):
    """The BASELINE cfg5 score in its literal order, sum_h w*relu(q.k*scale),
    in float64 (every e4m3 product and 128-term dot is exact there; the rest
    rounds at 2^-53, far below fp32), and sum_h |w*relu(.)|, which bounds the
    fp32 rounding of the oracle's factored form: its ~21 roundings (the int ->
    fp32 conversion, 16 fma per group, the group sums, the scale and the
    final product) each stay within 2^-24 of that sum."""
    tab = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).double()
    tab = torch.nan_to_num(tab, nan=0.0).numpy()
    kv = tab[k]
    T, S = q.shape[0], k.shape[0]
    real = np.empty((T, S))
    band = np.empty((T, S))
    for t in range(T):
        d = tab[q[t]] @ kv.T                              # [Hi, S], exact
        c = w[t][:, None].astype(np.float64) * np.maximum(d * scale[None, :].astype(np.float64), 0.0)
        real[t] = c.sum(0)
        band[t] = np.abs(c).sum(0)
        real[t, limit[t] + 1:] = -np.inf
    return real, band * 32 * 2.0 ** -24


@pytest.mark.parametrize("case", ["cfg5", "tie-stressed"])
def test_indexer_topk_sets_match_the_real_valued_score_up_to_fp32_rounding(case):
    """The oracle's exact fp32 score (one defined rounding order) selects the
    same top-k sets as the real-valued BASELINE formula, except for positions
    whose real score lies within the fp32 rounding band of the k-th largest
    one; ties (duplicated K rows) go to the lower position in both."""
    from dsa_amd import workloads
    if case == "cfg5":
        d = workloads.cfg5()
        q, k = d["q_idx"].numpy(), d["k_idx"].numpy()
        scale, w = d["k_scale"].numpy(), d["weights"].numpy()
        limit = d["causal_limit"].numpy().astype(np.int64)
        K = 2048
    else:
        q, k, scale, w, limit = _indexer_case(16, 64, 6000, seed=77, dup_rows=1500)
        K = 700
    sc = oracle.indexer_scores(q, k, scale, w, limit, 8)
    got = oracle.topk(sc, limit, K)
    real, eps = _real_scores_and_band(q, k, scale, w, limit)
    n_diff = 0
    for t in range(q.shape[0]):
        n = int(limit[t]) + 1
        order = np.lexsort((np.arange(n), -real[t, :n]))
        want = set(order[:K].tolist())
        have = set(got[t][got[t] >= 0].tolist())
        kth = order[K - 1]
        for s in want ^ have:
            n_diff += 1
            assert abs(real[t, s] - real[t, kth]) <= eps[t, s] + eps[t, kth], (case, t, s)
    # record how often the rounding band decides membership
    print(f"{case}: {n_diff} of {q.shape[0] * K} selected positions differ from the real-valued "
          f"top-{K}, all within the fp32 band of the k-th score")
    assert n_diff <= 0.001 * q.shape[0] * K
