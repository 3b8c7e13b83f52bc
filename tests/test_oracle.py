"""Pins the CPU oracle (oracle/oracle.cpp) before it is trusted as the checker.

Each test checks one oracle function against something that does not share
its code: the reference's own pq_utils.h compiled from /root/reference
(oracle/_ref) and the fixtures it wrote (tests/golden/ref_pq.npz), an
exact-rational restatement of the fused chains (tests/_exact.py), numpy brute
force, closed forms in float64, and invariants.
"""
import os

import numpy as np
import pytest

import oracle
from tests._exact import l2_fma_chain, lut_entry_chain, seq_sum_f32
from tests.golden.make_golden import inputs as golden_inputs

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_pq.npz")


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- distances
def test_l2_fma_matches_exact_fused_chain():
    rng = np.random.default_rng(1)
    for dim in (4, 17, 96, 128):
        for _ in range(3):
            a = rng.standard_normal(dim).astype(np.float32)
            b = rng.standard_normal(dim).astype(np.float32)
            assert _bits(oracle.l2_fma(a, b)) == _bits(l2_fma_chain(a, b))
            ref64 = float(np.sum((a.astype(np.float64) - b) ** 2))
            assert abs(oracle.l2_fma(a, b) - ref64) <= 1e-5 * ref64


@pytest.mark.parametrize("dim,m", [(128, 32), (128, 16), (96, 48), (96, 32)])
def test_lut_matches_exact_chain_and_closed_form(dim, m):
    rng = np.random.default_rng(dim * 100 + m)
    s = dim // m
    q = rng.standard_normal(dim).astype(np.float32)
    c = rng.standard_normal(dim).astype(np.float32)
    cb = rng.standard_normal((m, 256, s)).astype(np.float32)
    lut = oracle.lut(q, c, cb)
    r = (q - c).astype(np.float32)
    # closed form in float64 over the whole table: catches dropped terms, wrong index or transposes
    r64 = r.astype(np.float64).reshape(m, 1, s)
    ref64 = ((r64 - cb.astype(np.float64)) ** 2).sum(-1)
    np.testing.assert_allclose(lut, ref64, rtol=2e-6, atol=1e-7)
    # exact op order on a sample of entries (s=4 and s=8 special chains, generic otherwise)
    for sub, k in [(0, 0), (m - 1, 255), (m // 2, 17), (1, 128), (m - 2, 3)]:
        want = lut_entry_chain(r[sub * s:(sub + 1) * s], cb[sub, k])
        assert _bits(lut[sub, k]) == _bits(want), (sub, k)


def test_lut_chain_order_is_not_plain_rounding():
    # The fused chain must differ from separately rounded squares somewhere,
    # otherwise the exact-order checks above would be vacuous.
    rng = np.random.default_rng(7)
    q = rng.standard_normal(128).astype(np.float32)
    c = rng.standard_normal(128).astype(np.float32)
    cb = rng.standard_normal((32, 256, 4)).astype(np.float32)
    lut = oracle.lut(q, c, cb)
    d = ((q - c).reshape(32, 1, 4) - cb).astype(np.float32)
    plain = np.zeros((32, 256), np.float32)
    for j in range(4):
        plain = (plain + (d[..., j] * d[..., j]).astype(np.float32)).astype(np.float32)
    assert np.any(_bits(plain) != _bits(lut))


def test_adc_is_sequential_float32_sum():
    rng = np.random.default_rng(3)
    for m in (16, 32, 48):
        lut = (rng.random((m, 256)) * 3).astype(np.float32)
        for _ in range(5):
            code = rng.integers(0, 256, m).astype(np.uint8)
            want = seq_sum_f32(lut[np.arange(m), code])
            assert _bits(oracle.adc(code, lut)) == _bits(want)
            assert abs(oracle.adc(code, lut) - lut[np.arange(m), code].astype(np.float64).sum()) < 1e-4


# ---------------------------------------------------------------- coarse (A2, A3)
def _all_l2(q, c):
    return np.array([[oracle.l2_fma(a, b) for b in c] for a in q], np.float32)


def test_coarse_is_exact_ranking_with_tie_rule_and_prune():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((20, 32)).astype(np.float32)
    c = rng.standard_normal((40, 32)).astype(np.float32)
    c[7] = c[3]          # exact tie: list 3 must precede list 7
    c[25] = c[3]
    q[0] = c[3]          # distance exactly 0 for three lists
    ids, d = oracle.coarse(q, c, 9, prune_ratio=100.0)
    full = _all_l2(q, c)
    for i in range(q.shape[0]):
        order = np.lexsort((np.arange(40), full[i]))[:9]
        assert np.array_equal(d[i], full[i][order])
        best = full[i][order[0]]
        want = np.where(full[i][order] > np.float32(best * np.float32(100.0)), 0xFFFFFFFF, order).astype(np.uint32)
        assert np.array_equal(ids[i], want)
    # query 0 has best distance 0: everything with d > 0 is pruned
    assert list(ids[0][:3]) == [3, 7, 25] and np.all(ids[0][3:] == 0xFFFFFFFF)
    ids2, _ = oracle.coarse(q, c, 9, prune_ratio=1.5)
    assert np.any(ids2 == 0xFFFFFFFF)
    with pytest.raises(ValueError):
        oracle.coarse(q, c, 41)


def test_probe_counts():
    offsets = np.array([0, 5, 5, 12, 20], np.int32)
    probes = np.array([[0, 2, 0xFFFFFFFF], [1, 3, 2]], np.uint32)
    assert list(oracle.probe_counts(probes, offsets)) == [12, 15]


# ---------------------------------------------------------------- plain search (A4-A6, A10)
def _tiny_index(rng, n=500, dim=32, m=8, nlist=10):
    x = rng.standard_normal((n, dim)).astype(np.float32)
    cent = rng.standard_normal((nlist, dim)).astype(np.float32)
    assign = oracle.kmeans_assign(x, cent)
    cb = rng.standard_normal((m, 256, dim // m)).astype(np.float32) * 0.5
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    codes[10] = codes[11]  # identical codes in (possibly) the same list -> exact distance ties
    assign[11] = assign[10]
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    return x, cent, cb, offs, ids, lc


def test_search_plain_matches_brute_force():
    rng = np.random.default_rng(5)
    x, cent, cb, offs, ids, lc = _tiny_index(rng)
    q = rng.standard_normal((12, 32)).astype(np.float32)
    probes, _ = oracle.coarse(q, cent, 4)
    probes[3, 1] = 0xFFFFFFFF  # a pruned probe is skipped
    k = 15
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, k)
    for i in range(q.shape[0]):
        ds, vs = [], []
        for l in probes[i]:
            if l == 0xFFFFFFFF:
                continue
            lut = oracle.lut(q[i], cent[l], cb)
            m = cb.shape[0]
            for v in range(offs[l], offs[l + 1]):
                ds.append(seq_sum_f32(lut[np.arange(m), lc[v]]))
                vs.append(ids[v])
        ds, vs = np.array(ds, np.float32), np.array(vs, np.int32)
        order = np.lexsort((vs, ds))[:k]
        assert np.array_equal(oid[i][:len(order)], vs[order])
        assert np.array_equal(_bits(od[i][:len(order)]), _bits(ds[order]))
        assert np.all(oid[i][len(order):] == -1)


def test_search_plain_pads_short_results():
    rng = np.random.default_rng(6)
    x, cent, cb, offs, ids, lc = _tiny_index(rng, n=30, nlist=10)
    q = rng.standard_normal((2, 32)).astype(np.float32)
    probes = np.full((2, 2), 0xFFFFFFFF, np.uint32)
    probes[0, 0] = 0
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, 40)
    n0 = offs[1] - offs[0]
    assert np.all(oid[0][n0:] == -1) and np.all(od[0][n0:] == np.finfo(np.float32).max)
    assert np.all(oid[1] == -1)


# ---------------------------------------------------------------- k-means (A13, A14)
def test_kmeans_assign_is_argmin_lowest_index():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((300, 16)).astype(np.float32)
    c = rng.standard_normal((20, 16)).astype(np.float32)
    c[9] = c[4]
    x[0] = c[4]
    a = oracle.kmeans_assign(x, c)
    full = _all_l2(x, c)
    assert np.array_equal(a, np.argmin(full, axis=1))
    assert a[0] == 4


def test_kmeans_update_fixed_point_exact():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((1000, 8)).astype(np.float32)
    k = 7
    a = rng.integers(0, k - 1, 1000).astype(np.int32)  # cluster k-1 stays empty
    shift = oracle.fixed_shift(float(np.abs(x).max()), 1000)
    old = rng.standard_normal((k, 8)).astype(np.float32)
    for rule in (0, 1):
        got, cnt = oracle.kmeans_update(x, a, old, shift, rule)
        q = np.rint(np.ldexp(x.astype(np.float64), shift)).astype(np.int64)
        sums = np.zeros((k, 8), np.int64)
        np.add.at(sums, a, q)
        counts = np.bincount(a, minlength=k)
        assert np.array_equal(cnt, counts)
        want = old.copy() if rule == 1 else np.zeros_like(old)
        for c in range(k):
            if counts[c]:
                s = np.ldexp(sums[c].astype(np.float64), -shift).astype(np.float32)
                want[c] = (s * (np.float32(1.0) / np.float32(counts[c]))).astype(np.float32)
        assert np.array_equal(_bits(got), _bits(want))
        # the centroid is the member mean to float precision
        for c in range(k - 1):
            np.testing.assert_allclose(got[c], x[a == c].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)


def test_kmeans_init_strided_matches_mt19937():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((1000, 4)).astype(np.float32)
    k = 37
    cent, rows = oracle.kmeans_init_strided(x, k, 42)
    bg = np.random.MT19937()
    bg._legacy_seeding(42)
    raw = bg.random_raw(k).astype(np.int64)
    stride = max(1, 1000 // k)
    want = (np.arange(k) * stride + raw % stride) % 1000
    assert np.array_equal(rows, want)
    assert np.array_equal(cent, x[want])


def _mix64(z):
    M = (1 << 64) - 1
    z = (z + 0x9E3779B97F4A7C15) & M
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return z ^ (z >> 31)


def test_kmeans_init_pp_definition():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((200, 6)).astype(np.float32)
    k, seed = 9, 77
    cent, rows = oracle.kmeans_init_pp(x, k, seed)
    n = x.shape[0]
    r0 = _mix64(seed ^ _mix64(7)) % n
    want = [r0]
    d2 = np.array([oracle.l2_fma(v, x[r0]) for v in x], np.float32)
    mx = float(d2.max())
    e = int(np.frexp(mx)[1])
    lg = int(np.ceil(np.log2(n)))
    S = min(60, max(0, 62 - lg - e))
    for j in range(1, k):
        w = np.rint(np.ldexp(d2.astype(np.float64), S)).astype(np.uint64)
        tot = int(w.sum())
        u = _mix64(seed ^ _mix64(7) ^ _mix64(0x100000000 + j)) % tot
        pick = int(np.searchsorted(np.cumsum(w), u, side="right"))
        want.append(pick)
        d2 = np.minimum(d2, np.array([oracle.l2_fma(v, x[pick]) for v in x], np.float32))
    assert list(rows) == want
    assert len(set(want)) == k
    assert np.array_equal(cent, x[want])


def test_kmeans_init_pp_never_picks_a_covered_point():
    """D^2 seeding gives a point at distance 0 from a chosen centre weight 0:
    with k equal to the number of distinct rows (each repeated many times) the
    picks are exactly one row of each distinct value."""
    rng = np.random.default_rng(13)
    distinct = rng.standard_normal((12, 5)).astype(np.float32) * 3
    x = distinct[rng.integers(0, 12, 600)]
    x[:12] = distinct  # every value present
    for seed in (1, 2, 3, 99):
        cent, rows = oracle.kmeans_init_pp(x, 12, seed)
        got = {tuple(r) for r in np.asarray(cent)}
        assert len(got) == 12 and got == {tuple(r) for r in distinct}


def test_kmeans_init_pp_second_pick_follows_d2():
    """Across seeds, the second pick given the first is distributed as
    d^2 / sum d^2 (a chi-square bound that d or d^4 weights fail)."""
    x = np.array([[0.0], [1.0], [3.0], [7.0]], np.float32)
    counts = np.zeros((4, 4))
    for seed in range(4000):
        _, rows = oracle.kmeans_init_pp(x, 2, seed)
        counts[rows[0], rows[1]] += 1
    for r0 in range(4):
        n = counts[r0].sum()
        assert n > 500
        d2 = (x[:, 0] - x[r0, 0]) ** 2
        p = d2 / d2.sum()
        assert counts[r0, r0] == 0
        exp = n * p
        m = exp > 0
        chi2 = float((((counts[r0][m] - exp[m]) ** 2) / exp[m]).sum())
        assert chi2 < 16.3, (r0, counts[r0], exp)  # 3 cells, p < 0.001
        for alt in (np.sqrt(d2), d2 ** 2):  # the bound separates neighbouring weightings
            pa = alt / alt.sum()
            ea = n * pa
            ma = ea > 0
            assert float((((counts[r0][ma] - ea[ma]) ** 2) / ea[ma]).sum()) > 16.3


# ---------------------------------------------------------------- PQ (A15, A16) vs the reference's own code
def test_pq_against_golden_fixture():
    g = np.load(GOLDEN)
    km_data, x, cent, assign = golden_inputs()
    assert np.array_equal(_bits(oracle.pq_kmeans_fast(km_data, 256, 1234, 6)), _bits(g["kmeans_fast"]))
    cb = oracle.pq_train(x, assign, cent, 32, sample_size=500, iters=5)
    assert np.array_equal(_bits(cb), _bits(g["codebook"]))
    codes = oracle.pq_encode(x, assign, cent, g["codebook"], fma_mode=0)
    assert np.array_equal(codes, g["codes"])


@pytest.mark.skipif(oracle.ref_lib() is None, reason="oracle/_ref not built (needs /root/reference)")
def test_pq_against_reference_build():
    import ctypes
    ref = oracle.ref_lib()
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    rng = np.random.default_rng(13)
    data = rng.standard_normal((900, 4)).astype(np.float32) * 2
    out = np.empty((256, 4), np.float32)
    ref.ref_run_kmeans_pq_fast(P(data), 900, 4, 256, 4321, 4, P(out))
    assert np.array_equal(_bits(oracle.pq_kmeans_fast(data, 256, 4321, 4)), _bits(out))
    n, nlist = 800, 9
    cent = rng.standard_normal((nlist, 128)).astype(np.float32)
    a = rng.integers(0, nlist, n).astype(np.int32)
    x = (cent[a] + 0.2 * rng.standard_normal((n, 128))).astype(np.float32)
    cb = np.empty((32, 256, 4), np.float32)
    ref.ref_train_residual_pq_codebooks(P(x), n, P(a), P(cent), nlist, 700, 3, P(cb))
    assert np.array_equal(_bits(oracle.pq_train(x, a, cent, 32, sample_size=700, iters=3)), _bits(cb))
    codes = np.empty((n, 32), np.uint8)
    ref.ref_encode_residuals_to_pq(P(x), n, P(a), P(cent), nlist, P(cb), P(codes))
    assert np.array_equal(oracle.pq_encode(x, a, cent, cb, fma_mode=0), codes)


def test_pq_encode_fma_mode_is_argmin_of_fused_chain():
    rng = np.random.default_rng(14)
    n, dim, m = 40, 16, 4
    x = rng.standard_normal((n, dim)).astype(np.float32)
    cent = rng.standard_normal((3, dim)).astype(np.float32)
    a = rng.integers(0, 3, n).astype(np.int32)
    cb = rng.standard_normal((m, 256, 4)).astype(np.float32)
    cb[1, 200] = cb[1, 100]  # tie: lower codeword wins
    codes = oracle.pq_encode(x, a, cent, cb, fma_mode=1)
    for i in range(0, n, 7):
        r = (x[i] - cent[a[i]]).astype(np.float32)
        for sub in range(m):
            d = [l2_fma_chain(r[sub * 4:(sub + 1) * 4], cb[sub, k]) for k in range(256)]
            assert codes[i, sub] == int(np.argmin(np.array(d, np.float32)))


def test_pq_sample_is_mt19937_shuffle_prefix():
    rows = oracle.pq_sample(1000, 300)
    assert len(set(rows.tolist())) == 300 and rows.min() >= 0 and rows.max() < 1000
    assert len(oracle.pq_sample(100, 300)) == 100


# ---------------------------------------------------------------- lists (A17), kNN (A18)
def test_build_lists_round_trip():
    rng = np.random.default_rng(15)
    a = rng.integers(0, 6, 100).astype(np.int32)
    a[a == 4] = 5  # an empty list
    codes = rng.integers(0, 256, (100, 8)).astype(np.uint8)
    offs, ids, lc = oracle.build_lists(a, 6, codes)
    assert offs[0] == 0 and offs[-1] == 100 and offs[5] == offs[4]
    for l in range(6):
        seg = ids[offs[l]:offs[l + 1]]
        assert np.all(np.diff(seg) > 0) and np.all(a[seg] == l)
    assert np.array_equal(lc, codes[ids])


def test_knn_exact_brute_force():
    rng = np.random.default_rng(16)
    base = rng.standard_normal((300, 24)).astype(np.float32)
    base[50] = base[20]
    q = rng.standard_normal((5, 24)).astype(np.float32)
    q[1] = base[20]
    oid, od = oracle.knn_exact(q, base, 10)
    full = _all_l2(q, base)
    for i in range(5):
        order = np.lexsort((np.arange(300), full[i]))[:10]
        assert np.array_equal(oid[i], order) and np.array_equal(od[i], full[i][order])
    assert list(oid[1][:2]) == [20, 50]


# ---------------------------------------------------------------- generator
def test_gen_gmm_moments_and_determinism():
    a = oracle.gen_gmm(4000, 16, 4, seed=3, sig_lo=0.1)
    b = oracle.gen_gmm(4000, 16, 4, seed=3, sig_lo=0.1, nthreads=3)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, oracle.gen_gmm(4000, 16, 4, seed=3, set=1, sig_lo=0.1))
    assert a.min() > -1.0 - 0.8 and a.max() < 1.0 + 0.8
    # within-cluster spread ~ sigma: nearest of 4 centres explains the data
    from scipy.cluster.vq import kmeans2
    _, lab = kmeans2(a.astype(np.float64), 4, seed=0, minit="++")
    resid = np.concatenate([a[lab == j] - a[lab == j].mean(0) for j in range(4) if np.any(lab == j)])
    assert 0.08 < resid.std() < 0.2


# --------------------------------------------------------------------------- build_global's rebalancing queue
def _stub_split(rows, sub_k):
    """Deterministic stand-in for the local k-means: rows cut into sub_k contiguous parts, the first part
    carrying every row after a marker (to make a skewed child); centroid = the child's index."""
    parts = np.array_split(rows, sub_k)
    return [(p, np.float32(j)) for j, p in enumerate(parts)]


def test_rebalance_queue_order_and_thresholds():
    """build_global.cu:62-169 by hand: avg = 100 / 4 = 25, threshold (size_t)(2 avg) = 50, min 32.
    Initial buckets of sizes 10, 0, 60, 30: the empty one is dropped, 10 and 30 are final at once (in
    queue order), 60 splits into ceil(60 / 25) = 3 children of 20 appended behind them (FIFO)."""
    rows = np.arange(100, dtype=np.int32)
    buckets = [(rows[:10], 0), (rows[:0], 1), (rows[10:70], 2), (rows[70:], 3)]
    final, splits = oracle.rebalance_buckets(buckets, 100, 4, _stub_split)
    assert splits == 1
    assert [len(r) for r, _ in final] == [10, 30, 20, 20, 20]
    assert [c for _, c in final] == [0, 3, 0, 1, 2]
    assert np.array_equal(np.concatenate([r for r, _ in final]), np.r_[rows[:10], rows[70:], rows[10:70]])


def test_rebalance_resplits_oversized_children_at_the_back_of_the_queue():
    """A child still above the threshold is split again after the buckets queued before it; sub_k is at
    least 2 and at most size / 2; a bucket below 32 is final whatever its size against the threshold."""
    calls = []

    def split(rows, sub_k):
        calls.append((len(rows), sub_k))
        if len(rows) == 400:  # one heavy child of 300, the rest split evenly
            return [(rows[:300], 0), (rows[300:350], 1), (rows[350:], 2)]
        return [(p, j) for j, p in enumerate(np.array_split(rows, sub_k))]

    rows = np.arange(420, dtype=np.int32)
    # avg = 420 / 10 = 42, threshold 84
    final, splits = oracle.rebalance_buckets([(rows[:400], "a"), (rows[400:], "b")], 420, 10, split)
    # 400 -> sub_k ceil(400/42) = 10, then 300 -> ceil(300/42) = 8
    assert calls == [(400, 10), (300, 8)]
    assert splits == 2
    assert [len(r) for r, _ in final] == [20, 50, 50] + [38] * 4 + [37] * 4
    # the clamp: 33 rows with avg 1 (threshold 2) -> sub_k = min(33, 33 // 2) = 16
    calls.clear()
    oracle.rebalance_buckets([(np.arange(33, dtype=np.int32), 0)], 33, 33,
                             lambda r, k: calls.append((len(r), k)) or [(r[:0], 0)] * k)
    assert calls == [(33, 16)]
    # 31 rows above a threshold of 2 stay whole (below the 32-row minimum)
    final, splits = oracle.rebalance_buckets([(np.arange(31, dtype=np.int32), 0)], 31, 31, split)
    assert splits == 0 and len(final) == 1


def test_build_global_without_rebalancing_is_the_plain_build():
    x = oracle.gen_gmm(3000, 32, 8, seed=12, sig_lo=0.1)
    a = oracle.build_global(x, 16, 8, kmeans_iters=4, pq_iters=2, sample_size=1000, rebalance=False)
    b = oracle.build_ivfpq(x, 16, 8, kmeans_iters=4, pq_iters=2, sample_size=1000)
    for u, v in zip(a[:5], b):
        assert np.array_equal(np.asarray(u).view(np.uint8), np.asarray(v).view(np.uint8))
    assert a[5] == 0


def test_build_global_rebalancing_keeps_every_row_once():
    x = oracle.gen_gmm(6000, 32, 3, seed=13, sig_lo=0.05, sig_hi=0.3)
    offs, ids, codes, cent, cb, splits = oracle.build_global(x, 16, 8, kmeans_iters=3, pq_iters=2, sample_size=1000)
    L = offs.shape[0] - 1
    assert splits > 0 and L > 16 and cent.shape == (L, 32)
    assert np.array_equal(np.sort(ids), np.arange(6000))
    sizes = np.diff(offs)
    assert np.all((sizes <= int(6000 / 16 * 2)) | (sizes < 32)) and np.all(sizes > 0)
    lid = np.repeat(np.arange(L), sizes)
    assert np.all(np.diff(ids)[np.diff(lid) == 0] > 0)  # ascending inside each list
