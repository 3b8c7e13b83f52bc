"""Pins the oracle's restatement of the offline tuner (tune_parameters.cu:459-1053)
and checks the library's host-side tuner analytics (fgpu_tune_percentile*,
fgpu_tune_elbow) against it, on the CPU.

* orc_tune_list_stats: LUT entries against the fused chain evaluated in exact
  rational arithmetic with one correct rounding per step; on dyadic data (every
  operation exact) distances, ranks and k-th values against numpy brute force.
* orc_tune_coarse_order: numpy brute force with separately rounded float32
  products and sums (the reference's host code has no fused multiply-add).
* tune_percentile / tune_elbow: hand-worked known answers; the library's host
  functions equal them on random inputs.
"""
import ctypes
import math
import os
import subprocess
from fractions import Fraction

import numpy as np
import pytest

import oracle

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "fusiongpu_amd", "_lib",
                   "libfusiongpu.so")
BIN = os.path.join(os.path.dirname(LIB), "bin")


@pytest.fixture(scope="module")
def hostlib():
    l = ctypes.CDLL(LIB)
    l.fgpu_tune_elbow.restype = ctypes.c_int
    l.fgpu_tune_elbow.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.POINTER(ctypes.c_float)]
    l.fgpu_tune_percentile_int.restype = ctypes.c_int
    l.fgpu_tune_percentile_int.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_float]
    l.fgpu_tune_percentile.restype = ctypes.c_float
    l.fgpu_tune_percentile.argtypes = [ctypes.c_void_p, ctypes.c_longlong, ctypes.c_float]
    return l


def _round_f32(x: Fraction) -> np.float32:
    """Round a rational to the nearest float32, ties to even."""
    c = np.float32(float(x))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        err = abs(Fraction(float(cand)) - x)
        if best is None or err < best[0] or (err == best[0] and (cand.view(np.uint32) & 1) == 0):
            best = (err, cand)
    return best[1]


def _fma(a, b, c):
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _one_list_index(rng, n, dim, m, scale=None):
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    offsets = np.array([0, n], np.int32)
    ids = np.arange(n, dtype=np.int32)
    if scale is None:
        cent = rng.standard_normal((1, dim)).astype(np.float32)
        cb = (rng.standard_normal((m, 256, dim // m)) * 0.5).astype(np.float32)
    else:  # dyadic values: every product and sum below is exact in float32
        cent = (rng.integers(-4, 5, (1, dim)) * scale).astype(np.float32)
        cb = (rng.integers(-4, 5, (m, 256, dim // m)) * scale).astype(np.float32)
    return offsets, ids, codes, cent, cb


def test_tuner_lut_is_the_fused_chain():
    """pq_m = 1: a vector's PQ distance is one LUT entry, the sequential fused
    chain over the sub-vector of (q - c) - codeword (tune_parameters.cu:112-120)."""
    rng = np.random.default_rng(3)
    for dim in (4, 8, 2):
        offsets, ids, codes, cent, cb = _one_list_index(rng, 64, dim, 1)
        q = rng.standard_normal((1, dim)).astype(np.float32)
        tp, _, pr, _, _ = oracle.tune_list_stats(q, cent, cb, offsets, ids, codes, None, [0] * 64, [0] * 64,
                                                 list(range(64)))
        for j in range(64):
            acc = np.float32(0.0)
            for d in range(dim):
                r = np.float32(q[0, d] - cent[0, d])
                diff = np.float32(r - cb[0, codes[j, 0], d])
                acc = _fma(diff, diff, acc)
            assert tp[j].view(np.uint32) == acc.view(np.uint32), (dim, j)
        assert np.all(pr >= 1)


@pytest.mark.parametrize("dim,m", [(16, 4), (24, 8), (32, 32)])
def test_list_stats_brute_force_on_exact_data(dim, m):
    rng = np.random.default_rng(dim + m)
    n = 300
    offsets, ids, codes, cent, cb = _one_list_index(rng, n, dim, m, scale=0.25)
    codes[7] = codes[3]                          # equal PQ distances: strict rank
    base = (rng.integers(-4, 5, (n, dim)) * 0.25).astype(np.float32)
    base[9] = base[2]                            # equal exact distances
    q = (rng.integers(-4, 5, (2, dim)) * 0.25).astype(np.float32)
    S = dim // m
    r = (q[:, None, :] - cent[0][None, None, :]).reshape(2, 1, m, S)
    lut = ((r[:, :, :, None, :] - cb[None, None]) ** 2).sum(-1)[:, 0]          # [2][m][256], exact
    pq = lut[:, np.arange(m)[None, :], codes].sum(-1)                             # [2][n]
    ex = ((q[:, None, :] - base[None]) ** 2).sum(-1)                             # [2][n]
    targets = [3, 7, 9, 2, 150, 299, -1, 5000]
    pair_q = [0, 1, 0, 1, 0, 1, 0, 1]
    kth = [1, 10, 300, 301, 0, 50, 77, 2]
    tp, te, pr, er, kp = oracle.tune_list_stats(q, cent, cb, offsets, ids, codes, base, pair_q, [0] * 8, targets, kth)
    for p, (qi, t, k) in enumerate(zip(pair_q, targets, kth)):
        if 0 <= t < n:
            assert tp[p] == pq[qi, t] and te[p] == ex[qi, t]
            assert pr[p] == 1 + np.sum(pq[qi] < pq[qi, t]) and er[p] == 1 + np.sum(ex[qi] < ex[qi, t])
        else:
            assert pr[p] == 0 and er[p] == 0 and tp[p] == -1 and te[p] == -1
        if k > 0:
            assert kp[p] == np.sort(pq[qi])[min(k, n) - 1]
    # without raw vectors: no exact part; a pair outside the inputs: absent values
    _, te2, _, er2, _ = oracle.tune_list_stats(q, cent, cb, offsets, ids, codes, None, [0], [0], [3])
    assert te2[0] == -1 and er2[0] == 0
    tp3, _, pr3, _, kp3 = oracle.tune_list_stats(q, cent, cb, offsets, ids, codes, base, [5, 0], [0, 3], [3, 3],
                                                 [4, 4])
    assert np.all(pr3 == 0) and np.all(tp3 == -1) and np.all(kp3 == 0)


def test_coarse_order_is_host_form_sort():
    rng = np.random.default_rng(11)
    nl, dim = 57, 24
    cent = rng.standard_normal((nl, dim)).astype(np.float32)
    cent[40] = cent[12]                          # equal distances: the lower list id first
    q = rng.standard_normal((5, dim)).astype(np.float32)
    order, rank_of = oracle.tune_coarse_order(q, cent)
    for i in range(5):
        dist = np.zeros(nl, np.float32)
        for d in range(dim):
            diff = (q[i, d] - cent[:, d]).astype(np.float32)
            dist = (dist + (diff * diff).astype(np.float32)).astype(np.float32)
        want = np.lexsort((np.arange(nl), dist))
        assert np.array_equal(order[i], want)
        assert np.array_equal(rank_of[i][want], np.arange(1, nl + 1))
        assert rank_of[i][12] < rank_of[i][40]


def test_percentile_known_answers(hostlib):
    assert oracle.tune_percentile([5, 1, 3], 0.5) == 3           # sorted [1,3,5], floor(1.5) = 1
    assert oracle.tune_percentile([5, 1, 3], 0.995) == 5
    assert oracle.tune_percentile([7], 0.98) == 7
    assert oracle.tune_percentile([], 0.5) == 0
    assert oracle.tune_percentile(list(range(1000, 0, -1)), 0.995) == 996
    v = np.array([4, 9, 2, 2, 8], np.int32)
    assert hostlib.fgpu_tune_percentile_int(v.ctypes.data_as(ctypes.c_void_p), 5, 0.5) == 4
    assert hostlib.fgpu_tune_percentile_int(None, 0, 0.5) == 0
    f = np.array([0.5, 0.25, 2.0], np.float32)
    assert hostlib.fgpu_tune_percentile(f.ctypes.data_as(ctypes.c_void_p), 3, 0.99) == 2.0


def test_elbow_known_answers(hostlib):
    # fewer than 4 ranks: nothing is scored; the first coverage >= 0.6 wins
    assert oracle.tune_elbow([50, 20, 30], 100)[0] == 2
    assert oracle.tune_elbow([], 0)[0] == 1 and oracle.tune_elbow([0, 0], 0)[0] == 1
    # only rank 4 reaches 80% coverage inside the scored range (ranks 3..n-1)
    assert oracle.tune_elbow([30, 20, 20, 25, 5], 100)[0] == 4
    # a flat tail after a steep drop: rank 3 scores 8 * 0.83 (drop) + 3.98
    # (bonus) + ~0.5 (curvature); rank 4 ~4.4 (curvature) + 3.96; later ranks
    # only the bonus
    assert oracle.tune_elbow([500, 300, 50, 50, 50, 50, 50], 1050)[0] == 3
    for hits, tot in (([50, 20, 30], 100), ([30, 20, 20, 25, 5], 100), ([500, 300, 50, 50, 50, 50, 50], 1050)):
        h = np.array(hits, np.int32)
        cov = ctypes.c_float()
        got = hostlib.fgpu_tune_elbow(h.ctypes.data_as(ctypes.c_void_p), len(hits), tot, ctypes.byref(cov))
        want, wcov = oracle.tune_elbow(hits, tot)
        assert got == want and np.float32(cov.value) == wcov


def test_library_elbow_equals_oracle_on_random_hits(hostlib):
    rng = np.random.default_rng(0)
    for t in range(600):
        n = int(rng.integers(1, 45))
        if t % 3 == 0:
            hits = rng.integers(0, 60, n)
        elif t % 3 == 1:
            hits = (900 * np.exp(-rng.uniform(0.05, 1.2) * np.arange(n)) + rng.integers(0, 6, n)).astype(int)
        else:
            hits = np.sort(rng.integers(0, 300, n))[::-1]
        hits = np.ascontiguousarray(hits, np.int32)
        tot = int(hits.sum())
        cov = ctypes.c_float()
        got = hostlib.fgpu_tune_elbow(hits.ctypes.data_as(ctypes.c_void_p), n, tot, ctypes.byref(cov))
        want, wcov = oracle.tune_elbow(hits, tot)
        assert got == want and np.float32(cov.value) == wcov, hits.tolist()


def test_tool_usage_and_input_errors(tmp_path):
    tool = os.path.join(BIN, "tune_parameters")
    r = subprocess.run([tool], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "Usage" in r.stderr
    r = subprocess.run([tool, str(tmp_path / "none.fvecs")], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "cannot open" in r.stderr
    f = tmp_path / "d8.fvecs"
    rows = np.concatenate([np.full((4, 1), 8, np.int32).view(np.float32), np.zeros((4, 8), np.float32)], 1)
    f.write_bytes(rows.astype(np.float32).tobytes())
    r = subprocess.run([tool, str(f), "--bogus"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "unknown argument" in r.stderr
    r = subprocess.run([tool, str(f), "-k", "0"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1
    r = subprocess.run([tool, str(f), "--pq_m", "3"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "not a multiple" in r.stderr
    r = subprocess.run([tool, str(f), "--pq_m", "4", "--res", str(tmp_path)], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 1 and "ivf_data.bin" in r.stderr
