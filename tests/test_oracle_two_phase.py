"""Pins the oracle's two-phase search (A6-A10) and exact rerank (A11).

orc_search_two_phase is checked against orc_search_plain, which
test_oracle.py pins by brute force: on single lists it gives each list's
sorted distances, so the phase-1 cutoffs, the threshold and the candidate set
can be rebuilt in numpy from the reference's description
(gpu_global.cu:321-527, 852-867), and two parameter settings reduce the whole
search to plain top-k.  orc_rerank is checked against brute-force exact kNN
(orc_knn_exact, pinned in test_oracle.py) where its stop rule cannot fire,
and against hand-built candidate sequences whose stop point is worked out by
hand from gpu_global.cu:653-662.
"""
import numpy as np
import pytest

import oracle

FMAX = np.finfo(np.float32).max
PRUNED = 0xFFFFFFFF


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _index(rng, n=3000, dim=32, m=8, nlist=24, empty=(5,), big=7):
    p = rng.random(nlist) + 0.1
    for e in empty:
        p[e] = 0.0
    p[big] *= 12
    assign = rng.choice(nlist, size=n, p=p / p.sum()).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    codes[40] = codes[41]
    assign[41] = assign[40]
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = rng.standard_normal((nlist, dim)).astype(np.float32) * 0.7
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    return offs, ids, lc, cent, cb


def _list_sorted(q, cent, cb, offs, ids, lc, l):
    """(dists, ids) of list l sorted by the tie rule, from the pinned plain search."""
    n = int(offs[l + 1] - offs[l])
    probe = np.array([[l]], np.uint32)
    oid, od = oracle.search_plain(q[None], cent, cb, offs, ids, lc, probe, max(n, 1))
    return od[0, :n], oid[0, :n]


def _expected(q, cent, cb, offs, ids, lc, probes, p1_lists, limit_k, coeff, rerank_m):
    nlist = cent.shape[0]
    nprobe = probes.shape[0]
    p1 = max(0, min(nprobe, p1_lists))
    cand_d, cand_i, cuts = [], [], []
    for j in range(p1):
        l = int(probes[j])
        if l >= nlist or offs[l + 1] == offs[l]:
            cuts.append(np.float32(0.0))
            continue
        d, i = _list_sorted(q, cent, cb, offs, ids, lc, l)
        w = min(len(d), limit_k)
        cand_d += list(d[:w])
        cand_i += list(i[:w])
        cuts.append(d[w - 1])
    pos = [c for c in cuts if c > 0]
    thr = np.float32(np.float32(min(pos)) * np.float32(coeff)) if pos else FMAX
    for j in range(p1, nprobe):
        l = int(probes[j])
        if l >= nlist:
            continue
        d, i = _list_sorted(q, cent, cb, offs, ids, lc, l)
        keep = d <= thr
        cand_d += list(d[keep])
        cand_i += list(i[keep])
    cand_d, cand_i = np.array(cand_d, np.float32), np.array(cand_i, np.int32)
    order = np.lexsort((cand_i, cand_d))[:rerank_m]
    return cand_d[order], cand_i[order], np.array(cuts, np.float32), thr


@pytest.mark.parametrize("p1_lists,limit_k,coeff", [(3, 5, 1.0), (4, 1, 1.5), (2, 64, 0.5), (6, 10, 0.0)])
def test_two_phase_matches_composition_of_single_lists(p1_lists, limit_k, coeff):
    rng = np.random.default_rng(p1_lists * 100 + limit_k)
    offs, ids, lc, cent, cb = _index(rng)
    q = rng.standard_normal((10, 32)).astype(np.float32) * 0.7
    probes, _ = oracle.coarse(q, cent, 8)
    probes[2, 1] = PRUNED                      # a pruned phase-1 probe -> cutoff 0
    probes[3, 0] = 5                           # an empty list first
    probes[4, 6] = 99                          # out-of-range id counts as pruned
    rerank_m = 60
    oid, od, cnt, cut, thr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1_lists, limit_k, coeff,
                                                     rerank_m)
    for i in range(q.shape[0]):
        wd, wi, wcut, wthr = _expected(q[i], cent, cb, offs, ids, lc, probes[i], p1_lists, limit_k, coeff, rerank_m)
        c = len(wd)
        assert cnt[i] == c
        assert np.array_equal(oid[i, :c], wi) and np.array_equal(_bits(od[i, :c]), _bits(wd))
        assert np.all(oid[i, c:] == -1) and np.all(od[i, c:] == FMAX)
        assert np.array_equal(_bits(cut[i]), _bits(wcut))
        assert _bits(thr[i]) == _bits(wthr)
    assert np.all(cut[2, 1] == 0) and cut[3, 0] == 0


def test_two_phase_reduces_to_plain_search():
    rng = np.random.default_rng(3)
    offs, ids, lc, cent, cb = _index(rng)
    q = rng.standard_normal((8, 32)).astype(np.float32) * 0.7
    probes, _ = oracle.coarse(q, cent, 6)
    longest = int(np.diff(offs).max())
    for rerank_m in (1, 17, 200):
        pid, pd = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, rerank_m)
        # every list is phase 1 and keeps all of its vectors
        a = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, 6, longest, 1.0, rerank_m)
        # no phase 1 at all: no cutoff, thr = FLT_MAX, every vector passes phase 2
        b = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, 0, 10, 1.0, rerank_m)
        for oid, od, cnt, _, thr in (a, b):
            assert np.array_equal(oid, pid) and np.array_equal(_bits(od), _bits(pd))
        assert np.all(b[4] == FMAX) and b[3].shape == (8, 0)


def test_two_phase_threshold_filters_phase_two():
    rng = np.random.default_rng(4)
    offs, ids, lc, cent, cb = _index(rng)
    q = rng.standard_normal((6, 32)).astype(np.float32) * 0.7
    probes, _ = oracle.coarse(q, cent, 8)
    # coeff 0: the threshold is 0, so only phase-1 candidates remain (no ADC distance is 0 here)
    oid, od, cnt, cut, thr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, 3, 7, 0.0, 500)
    assert np.all(thr == 0.0)
    for i in range(6):
        nonempty = sum(1 for l in probes[i, :3] if offs[l + 1] > offs[l])
        want = sum(min(7, int(offs[l + 1] - offs[l])) for l in probes[i, :3])
        assert cnt[i] == want and nonempty > 0
    # a larger coefficient can only add candidates, never drop one
    _, _, cnt2, _, _ = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, 3, 7, 2.0, 5000)
    assert np.all(cnt2 >= cnt)


# ---------------------------------------------------------------- rerank (A11)
def _knn_subset(q, base, cand, k):
    sub = np.unique(cand[cand >= 0])
    kid, kd = oracle.knn_exact(q[None], base[sub], k)
    kid = np.where(kid[0] >= 0, sub[np.maximum(kid[0], 0)], -1)
    return kid, kd[0]


def test_rerank_never_stable_is_exact_top_k_of_all_candidates():
    rng = np.random.default_rng(12)
    base = rng.standard_normal((2000, 24)).astype(np.float32)
    q = rng.standard_normal((5, 24)).astype(np.float32)
    rm, k = 300, 20
    cand = np.stack([rng.permutation(2000)[:rm] for _ in range(5)]).astype(np.int32)
    counts = np.array([300, 250, 21, 5, 0], np.int32)
    oid, od, vis = oracle.rerank(q, base, cand, counts, k, mb=32, eps=-1.0, beta=2)
    for i in range(5):
        c = counts[i]
        wid, wd = _knn_subset(q[i], base, cand[i, :c], k) if c else (np.full(k, -1), np.full(k, FMAX, np.float32))
        assert np.array_equal(oid[i], wid)
        assert np.array_equal(_bits(od[i]), _bits(wd))
        assert vis[i] == c
    assert np.all(oid[3, 5:] == -1) and np.all(od[4] == FMAX)


def test_rerank_always_stable_stops_after_one_batch():
    rng = np.random.default_rng(13)
    base = rng.standard_normal((500, 16)).astype(np.float32)
    q = rng.standard_normal((3, 16)).astype(np.float32)
    cand = np.stack([rng.permutation(500)[:100] for _ in range(3)]).astype(np.int32)
    counts = np.array([100, 100, 7], np.int32)
    oid, od, vis = oracle.rerank(q, base, cand, counts, 5, mb=16, eps=1.0, beta=1)
    assert list(vis) == [16, 16, 7]
    for i in range(3):
        wid, wd = _knn_subset(q[i], base, cand[i, :min(16, counts[i])], 5)
        assert np.array_equal(oid[i], wid) and np.array_equal(_bits(od[i]), _bits(wd))


def test_rerank_stop_rule_hand_worked():
    # q = 0; base row j = (a_j, 0) so the exact distance is a_j^2, an integer.
    a = np.array([2, 3, 1, 4, 5, 6, 0, 7], np.float32)
    base = np.stack([a, np.zeros_like(a)], 1).astype(np.float32)
    q = np.zeros((1, 2), np.float32)
    cand = np.arange(8, dtype=np.int32)[None]
    # k = 2, mb = 2, eps = 0.5, beta = 2:
    #   batch {0,1} (d 4, 9): top {0,1}, chg 2 -> 1.0 > 0.5, stable 0
    #   batch {2,3} (d 1,16): top {2,0}, chg 1 -> 0.5 <= 0.5, stable 1
    #   batch {4,5} (d25,36): top {2,0}, chg 0 -> stable 2 >= beta: stop
    # row 6 (d 0) is never evaluated.
    oid, od, vis = oracle.rerank(q, base, cand, np.array([8], np.int32), 2, mb=2, eps=0.5, beta=2)
    assert list(oid[0]) == [2, 0] and list(od[0]) == [1.0, 4.0] and vis[0] == 6
    # beta = 3 needs one more stable batch: {6,7} brings row 6 (d 0) in, chg 1 -> stable 3: stop
    oid, od, vis = oracle.rerank(q, base, cand, np.array([8], np.int32), 2, mb=2, eps=0.5, beta=3)
    assert list(oid[0]) == [6, 2] and list(od[0]) == [0.0, 1.0] and vis[0] == 8
    # eps = 0.4 < 1/2: any change resets; the walk only ends when candidates run out
    oid, od, vis = oracle.rerank(q, base, cand, np.array([8], np.int32), 2, mb=2, eps=0.4, beta=2)
    assert list(oid[0]) == [6, 2] and vis[0] == 8


def test_rerank_skips_invalid_ids_and_keeps_duplicates():
    base = np.arange(20, dtype=np.float32).reshape(10, 2)
    q = np.zeros((1, 2), np.float32)
    cand = np.array([[3, -1, 3, 57, 1, 2]], np.int32)
    oid, od, vis = oracle.rerank(q, base, cand, np.array([6], np.int32), 4, mb=8, eps=-1.0, beta=2)
    # rows 1 (d 4+9=13), 2 (16+25=41), 3 twice (36+49=85); -1 and 57 are skipped
    assert list(oid[0]) == [1, 2, 3, 3] and list(od[0]) == [13.0, 41.0, 85.0, 85.0] and vis[0] == 6


def test_two_phase_threshold_is_inclusive():
    # List 1 is list 0 again (same centroid, same codes, other ids), so the
    # phase-1 cutoff of list 0 reappears exactly in phase 2 (gpu_global.cu:482: dist <= threshold).
    rng = np.random.default_rng(21)
    n0, m, dim = 50, 8, 32
    codes0 = rng.integers(0, 256, (n0, m)).astype(np.uint8)
    lc = np.concatenate([codes0, codes0])
    ids = np.arange(2 * n0, dtype=np.int32)
    offs = np.array([0, n0, 2 * n0, 2 * n0], np.int32)
    cent = rng.standard_normal((3, dim)).astype(np.float32)
    cent[1] = cent[0]
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    q = cent[:1] + np.float32(0.1)
    probes = np.array([[0, 1]], np.uint32)
    oid, od, cnt, cut, thr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, 1, 3, 1.0, 10)
    d0, i0 = _list_sorted(q[0], cent, cb, offs, ids, lc, 0)
    assert _bits(thr[0]) == _bits(d0[2]) and len(set(d0[:4].tolist())) == 4
    assert cnt[0] == 6                           # 3 from phase 1 + 3 at or below the cutoff in phase 2
    assert sorted(oid[0, :6].tolist()) == sorted(i0[:3].tolist() + (i0[:3] + n0).tolist())


def _pre_cut(q, cent, cb, offs, ids, lc, probes, p1_lists, limit_k, coeff):
    """Candidates before the rerank_m cut, rebuilt from single lists: every
    phase-1 list's min(n, limit_k) plus every phase-2 vector with d <= thr."""
    nlist = cent.shape[0]
    _, _, _, thr = _expected(q, cent, cb, offs, ids, lc, probes, p1_lists, limit_k, coeff, 1)
    p1 = max(0, min(probes.shape[0], p1_lists))
    n = 0
    for j, l in enumerate(int(v) for v in probes):
        if l >= nlist or offs[l + 1] == offs[l]:
            continue
        if j < p1:
            n += min(int(offs[l + 1] - offs[l]), limit_k)
        else:
            d, _ = _list_sorted(q, cent, cb, offs, ids, lc, l)
            n += int((d <= thr).sum())
    return n


@pytest.mark.parametrize("p1_lists,limit_k,coeff", [(3, 5, 1.0), (4, 1, 1.5), (8, 10, 1.0), (0, 10, 1.0)])
def test_two_phase_pre_cut_counts(p1_lists, limit_k, coeff):
    """The count the reference accumulates per query before the rerank_m cut
    (query_atomic_counters, gpu_global.cu:349, 493-526): rebuilt from single
    lists, the same for every rerank_m, and equal to the kept count once
    rerank_m holds them all."""
    rng = np.random.default_rng(p1_lists * 10 + limit_k + 7)
    offs, ids, lc, cent, cb = _index(rng)
    q = rng.standard_normal((8, 32)).astype(np.float32) * 0.7
    probes, _ = oracle.coarse(q, cent, 8)
    probes[1, 2] = PRUNED
    probes[2, 0] = 5                           # an empty list
    pres = []
    for rerank_m in (1, 17, 4000):
        *_, pre = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1_lists, limit_k, coeff, rerank_m,
                                          want_pre_cut=True)
        pres.append(pre)
        if rerank_m == 4000:
            cnt = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1_lists, limit_k, coeff, rerank_m)[2]
            assert np.array_equal(cnt, pre)
    assert np.array_equal(pres[0], pres[1]) and np.array_equal(pres[0], pres[2])
    for i in range(q.shape[0]):
        assert pres[0][i] == _pre_cut(q[i], cent, cb, offs, ids, lc, probes[i], p1_lists, limit_k, coeff)


def test_rerank_state_hand_worked():
    """stab[] and fin[] as run_gpu_rerank leaves them (gpu_global.cu:603-609,
    615, 653-662), on the hand-worked sequence above."""
    a = np.array([2, 3, 1, 4, 5, 6, 0, 7], np.float32)
    base = np.stack([a, np.zeros_like(a)], 1).astype(np.float32)
    q = np.zeros((1, 2), np.float32)
    cand = np.arange(8, dtype=np.int32)[None]

    def state(count, eps, beta):
        *_, stab, fin = oracle.rerank(q, base, cand, np.array([count], np.int32), 2, mb=2, eps=eps, beta=beta,
                                      want_state=True)
        return int(stab[0]), int(fin[0])

    assert state(8, 0.5, 2) == (2, 1)    # stops on stability after batch {4,5}
    assert state(8, 0.5, 3) == (3, 1)    # one batch later
    # eps 0.4: the last batch {6,7} changes one of two -> stable 0; offsets 0..6 all run, none past the
    # candidates before rm = 8, so fin stays false
    assert state(8, 0.4, 2) == (0, 0)
    # five candidates: {0,1} chg 2, {2,3} chg 1, {4} chg 0 -> stable 1; offset 6 >= 5 -> finished
    assert state(5, 0.4, 2) == (1, 1)
    assert state(0, 0.4, 2) == (0, 1)    # offset 0 >= 0 candidates


def test_rerank_state_never_stable():
    rng = np.random.default_rng(14)
    base = rng.standard_normal((400, 8)).astype(np.float32)
    q = rng.standard_normal((5, 8)).astype(np.float32)
    rm, mb = 64, 16
    cand = np.stack([rng.permutation(400)[:rm] for _ in range(5)]).astype(np.int32)
    counts = np.array([64, 63, 48, 1, 0], np.int32)
    *_, stab, fin = oracle.rerank(q, base, cand, counts, 4, mb=mb, eps=-1.0, beta=2, want_state=True)
    assert np.all(stab == 0)
    # finished exactly when an offset below rm lies at or past the candidates
    assert list(fin) == [int(-(-c // mb) * mb < rm) for c in counts] == [0, 0, 1, 1, 1]
