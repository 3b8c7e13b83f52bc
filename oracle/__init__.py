"""CPU oracle for parity tests -- TEST INFRASTRUCTURE ONLY.

ctypes wrappers over oracle/liboracle.so (oracle.cpp, the CPU restatement of
the reference's search and build path) and, when built, oracle/_ref/libref.so
(the reference's own pq_utils.h/utils.h compiled from /root/reference).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
package, and only as the checker or the timed CPU baseline.
"""
from __future__ import annotations

import collections
import ctypes
import math
import os

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(_DIR, "liboracle.so")
REF_SO = os.path.join(_DIR, "_ref", "libref.so")

_c = ctypes
_vp, _i32, _i64, _u64, _f32, _f64, _u32 = (_c.c_void_p, _c.c_int, _c.c_longlong, _c.c_ulonglong, _c.c_float,
                                           _c.c_double, _c.c_uint)


def _p(a):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_vp)


_SIGS = {
    "orc_max_threads": (_i32, []),
    "orc_gen_gmm": (None, [_i64, _i32, _i32, _f64, _f64, _f64, _f64, _u64, _i32, _vp, _i32]),
    "orc_l2_fma": (_f32, [_vp, _vp, _i32]),
    "orc_lut": (None, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "orc_adc": (_f32, [_vp, _vp, _i32]),
    "orc_coarse": (_i32, [_vp, _i32, _vp, _i32, _i32, _i32, _f32, _vp, _vp, _i32]),
    "orc_probe_counts": (None, [_vp, _i32, _i32, _vp, _vp]),
    "orc_search_plain": (None, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _vp, _vp, _i32]),
    "orc_knn_exact": (None, [_vp, _i32, _vp, _i64, _i32, _i32, _vp, _vp, _i32]),
    "orc_search_two_phase": (None, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i32, _i32, _i32,
                                    _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32]),
    "orc_rerank": (None, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp, _vp, _vp,
                          _i32]),
    "orc_graph_search": (None, [_vp, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _u64, _vp, _vp, _vp,
                                _i32]),
    "orc_kmeans_assign": (None, [_vp, _i64, _vp, _i32, _i32, _vp, _i32]),
    "orc_fixed_shift": (_i32, [_f32, _i64]),
    "orc_kmeans_update": (None, [_vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "orc_kmeans_init_strided": (None, [_vp, _i64, _i32, _i32, _u32, _vp, _vp]),
    "orc_kmeans_init_pp": (None, [_vp, _i64, _i32, _i32, _u64, _vp, _vp, _i32]),
    "orc_pq_kmeans_fast": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _vp]),
    "orc_pq_sample": (_i32, [_i64, _i32, _vp]),
    "orc_pq_train": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp, _i32, _i32, _vp, _i32]),
    "orc_pq_encode": (None, [_vp, _i64, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _i32]),
    "orc_build_lists": (None, [_vp, _i64, _i32, _vp, _i32, _vp, _vp, _vp]),
    "orc_tune_list_stats": (None, [_vp, _i32, _i32, _vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                                   _vp, _i32, _vp, _vp, _vp, _vp, _vp, _i32]),
    "orc_tune_coarse_order": (None, [_vp, _i32, _vp, _i32, _i32, _vp, _vp, _i32]),
}


def _load():
    if not os.path.exists(ORACLE_SO):
        raise ImportError(f"{ORACLE_SO} not built; run `make -C oracle`")
    l = ctypes.CDLL(ORACLE_SO)
    for name, (res, args) in _SIGS.items():
        f = getattr(l, name)
        f.restype = res
        f.argtypes = args
    return l


lib = _load()


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def i32(a):
    return np.ascontiguousarray(a, np.int32)


def u8(a):
    return np.ascontiguousarray(a, np.uint8)


def gen_gmm(n, dim, ncomp, seed, set=0, lo=-1.0, hi=1.0, sig_lo=0.1, sig_hi=None, nthreads=0):
    out = np.empty((n, dim), np.float32)
    lib.orc_gen_gmm(n, dim, ncomp, lo, hi, sig_lo, sig_lo if sig_hi is None else sig_hi, seed, set, _p(out), nthreads)
    return out


def l2_fma(a, b):
    a, b = f32(a), f32(b)
    return lib.orc_l2_fma(_p(a), _p(b), a.shape[0])


def lut(q, c, codebook):
    q, c, codebook = f32(q), f32(c), f32(codebook)
    m = codebook.shape[0]
    out = np.empty((m, 256), np.float32)
    lib.orc_lut(_p(q), _p(c), _p(codebook), q.shape[0], m, _p(out))
    return out


def adc(code, lut_):
    code, lut_ = u8(code), f32(lut_)
    return lib.orc_adc(_p(code), _p(lut_), code.shape[0])


def coarse(q, cent, nprobe, prune_ratio=100.0, nthreads=0):
    q, cent = f32(q), f32(cent)
    nq, dim = q.shape
    ids = np.empty((nq, nprobe), np.uint32)
    d = np.empty((nq, nprobe), np.float32)
    rc = lib.orc_coarse(_p(q), nq, _p(cent), cent.shape[0], dim, nprobe, prune_ratio, _p(ids), _p(d), nthreads)
    if rc != 0:
        raise ValueError("orc_coarse: bad arguments")
    return ids, d


def probe_counts(probe_ids, offsets):
    probe_ids = np.ascontiguousarray(probe_ids, np.uint32)
    offsets = i32(offsets)
    nq, nprobe = probe_ids.shape
    out = np.empty(nq, np.int32)
    lib.orc_probe_counts(_p(probe_ids), nq, nprobe, _p(offsets), _p(out))
    return out


def search_plain(q, cent, codebook, offsets, ids, codes, probe_ids, k, nthreads=0):
    q, cent, codebook, offsets, ids, codes = f32(q), f32(cent), f32(codebook), i32(offsets), i32(ids), u8(codes)
    probe_ids = np.ascontiguousarray(probe_ids, np.uint32)
    nq, dim = q.shape
    m = codebook.shape[0]
    oid = np.empty((nq, k), np.int32)
    od = np.empty((nq, k), np.float32)
    lib.orc_search_plain(_p(q), nq, dim, m, _p(cent), _p(codebook), _p(offsets), _p(ids), _p(codes), _p(probe_ids),
                         probe_ids.shape[1], k, _p(oid), _p(od), nthreads)
    return oid, od


def search_two_phase(q, cent, codebook, offsets, ids, codes, probe_ids, p1_lists, limit_k, threshold_coeff, rerank_m,
                     nthreads=0, want_pre_cut=False):
    """run_gpu_batch_logic restated: (top_ids [nq][rerank_m], top_dists, counts [nq], cutoffs [nq][p1], thr [nq])
    and, with want_pre_cut, each query's candidate count before the rerank_m cut (the reference's d_atomic)."""
    q, cent, codebook, offsets, ids, codes = f32(q), f32(cent), f32(codebook), i32(offsets), i32(ids), u8(codes)
    probe_ids = np.ascontiguousarray(probe_ids, np.uint32)
    nq, dim = q.shape
    nprobe = probe_ids.shape[1]
    p1 = max(0, min(nprobe, p1_lists))
    oid = np.empty((nq, rerank_m), np.int32)
    od = np.empty((nq, rerank_m), np.float32)
    cnt = np.empty(nq, np.int32)
    cut = np.empty((nq, max(p1, 1)), np.float32)
    thr = np.empty(nq, np.float32)
    pre = np.empty(nq, np.int32)
    lib.orc_search_two_phase(_p(q), nq, dim, codebook.shape[0], _p(cent), _p(codebook), _p(offsets), _p(ids),
                             _p(codes), cent.shape[0], _p(probe_ids), nprobe, p1_lists, limit_k, threshold_coeff,
                             rerank_m, _p(oid), _p(od), _p(cnt), _p(cut), _p(thr), _p(pre), nthreads)
    if want_pre_cut:
        return oid, od, cnt, cut[:, :p1], thr, pre
    return oid, od, cnt, cut[:, :p1], thr


def rerank(q, base, cand_ids, counts, k, mb=128, eps=0.1, beta=2, nthreads=0, want_state=False):
    """run_gpu_rerank restated: (ids [nq][k], dists [nq][k], visited [nq]) and, with want_state, the
    reference's stab[] (int32) and fin[] (uint8) as it leaves them."""
    q, base, cand_ids, counts = f32(q), f32(base), i32(cand_ids), i32(counts)
    nq, dim = q.shape
    rm = cand_ids.shape[1]
    oid = np.empty((nq, k), np.int32)
    od = np.empty((nq, k), np.float32)
    vis = np.empty(nq, np.int32)
    stab = np.empty(nq, np.int32)
    fin = np.empty(nq, np.uint8)
    lib.orc_rerank(_p(q), nq, dim, _p(base), base.shape[0], _p(cand_ids), _p(counts), rm, k, mb, eps, beta, _p(oid),
                   _p(od), _p(vis), _p(stab), _p(fin), nthreads)
    if want_state:
        return oid, od, vis, stab, fin
    return oid, od, vis


def knn_exact(q, base, k, nthreads=0):
    q, base = f32(q), f32(base)
    oid = np.empty((q.shape[0], k), np.int32)
    od = np.empty((q.shape[0], k), np.float32)
    lib.orc_knn_exact(_p(q), q.shape[0], _p(base), base.shape[0], q.shape[1], k, _p(oid), _p(od), nthreads)
    return oid, od


# ---------------------------------------------------------------------------- tuner (tune_parameters.cu:459-1053)

def tune_list_stats(q, cent, codebook, offsets, ids, codes, base, pair_q, pair_l, pair_t=None, pair_k=None,
                    nthreads=0):
    """Per (query, list) pair: target PQ/exact distance and ranks, and the k-th PQ distance (orc_tune_list_stats)."""
    q, cent, codebook = f32(q), f32(cent), f32(codebook)
    offsets, ids, codes = i32(offsets), i32(ids), u8(codes)
    pair_q, pair_l = i32(pair_q), i32(pair_l)
    npairs = pair_q.shape[0]
    m = codebook.shape[0]
    tp, te = np.empty(npairs, np.float32), np.empty(npairs, np.float32)
    pr, er = np.empty(npairs, np.int32), np.empty(npairs, np.int32)
    kp = np.empty(npairs, np.float32)
    pt = i32(pair_t) if pair_t is not None else None
    pk = i32(pair_k) if pair_k is not None else None
    b = f32(base) if base is not None else None
    lib.orc_tune_list_stats(_p(q), q.shape[0], q.shape[1], _p(cent), cent.shape[0], _p(codebook), m, _p(offsets),
                            _p(ids), _p(codes), _p(b) if b is not None else None, b.shape[0] if b is not None else 0,
                            _p(pair_q), _p(pair_l), _p(pt) if pt is not None else None,
                            _p(pk) if pk is not None else None, npairs, _p(tp), _p(te), _p(pr), _p(er), _p(kp),
                            nthreads)
    return tp, te, pr, er, kp


def tune_coarse_order(q, cent, nthreads=0):
    """The tuner's host-form coarse order: (order [nq][nlist], rank_of [nq][nlist], 1-based)."""
    q, cent = f32(q), f32(cent)
    nq, nl = q.shape[0], cent.shape[0]
    order = np.empty((nq, nl), np.int32)
    rank_of = np.empty((nq, nl), np.int32)
    lib.orc_tune_coarse_order(_p(q), nq, _p(cent), nl, q.shape[1], _p(order), _p(rank_of), nthreads)
    return order, rank_of


def tune_percentile(values, pct):
    """compute_percentile(_int) (tune_parameters.cu:170-183): sorted[floor(n * pct)] with the product in float32,
    clamped; 0 for an empty sample."""
    v = np.sort(np.asarray(values))
    if v.size == 0:
        return 0
    idx = int(np.float32(v.size) * np.float32(pct))
    return v[min(idx, v.size - 1)]


_libm = ctypes.CDLL("libm.so.6")
_libm.logf.restype, _libm.logf.argtypes = _f32, [_f32]


def _f(x):
    return np.float32(x)


def tune_elbow(hits, total_hits):
    """find_elbow_point (tune_parameters.cu:199-456), float32 throughout as the reference's host code; log via the C
    library's logf.  Returns (elbow list count, coverage there)."""
    hits = [int(h) for h in hits]
    n = len(hits)
    if n == 0 or total_hits == 0:
        return 1, _f(0.0)
    cov, lg = [], []
    cum = 0
    for h in hits:
        cum += h
        cov.append(_f(_f(cum) / _f(total_hits)))
        lg.append(_f(_libm.logf(float(_f(h) + _f(1.0)))))
    sm = []
    for i in range(n):
        if i == 0 or i == n - 1:
            sm.append(lg[i])
        else:
            sm.append(_f(_f(_f(_f(0.25) * lg[i - 1]) + _f(_f(0.5) * lg[i])) + _f(_f(0.25) * lg[i + 1])))
    curv = [_f(0.0)] * n
    for i in range(1, n - 1):
        curv[i] = _f(_f(sm[i + 1] - _f(_f(2.0) * sm[i])) + sm[i - 1])
    vol = [0.0] * n
    for i in range(1, n - 1):
        d1, d2 = _f(hits[i - 1] - hits[i]), _f(hits[i] - hits[i + 1])
        if _f(d1 * d2) < 0:
            vol[i] = 1.0
    best, best_score = -1, _f(-1e9)
    i = 2
    while i + 1 < n and i < 30:
        if cov[i] >= _f(0.60):
            cs = _f(abs(curv[i]) * _f(10.0))
            db = _f(_f(hits[i - 1] - hits[i]) / _f(_f(hits[i - 1]) + _f(1.0)))
            da = _f(_f(hits[i] - hits[i + 1]) / _f(_f(hits[i]) + _f(1.0)))
            ds = _f(_f(db - da) * _f(8.0)) if da < db else _f(0.0)
            pen = _f(_f(vol[i]) * _f(5.0))
            r = _f(_f(i) / _f(32.0))
            bonus = _f(_f(4.0) * _f(_f(1.0) - _f(r * r)))
            score = _f(_f(_f(cs + ds) + bonus) - pen)
            if cov[i] >= _f(0.80) and score > best_score:
                best_score, best = score, i
        i += 1
    if best >= 0:
        return best + 1, cov[best]
    for i in range(n):
        if cov[i] >= _f(0.60):
            return i + 1, cov[i]
    return 1, _f(0.0)


def tune_parameters(base, offsets, ids, codes, cent, codebook, samples, k):
    """The tuner's recommendations (tune_search_parameters, tune_parameters.cu:459-1012) for the given sampled base
    rows: (top_m, p1_lists, limit_k, threshold_coeff)."""
    base = f32(base)
    offsets, ids = i32(offsets), i32(ids)
    nl = offsets.shape[0] - 1
    q = np.ascontiguousarray(base[np.asarray(samples)])
    nq = q.shape[0]
    gt, _ = knn_exact(q, base, k)
    list_of = {}
    for c in range(nl):
        for j in range(offsets[c], offsets[c + 1]):
            list_of.setdefault(int(ids[j]), c)
    order, rank_of = tune_coarse_order(q, cent)
    ranks = [int(rank_of[i, list_of[int(t)]]) for i in range(nq) for t in gt[i] if int(t) in list_of]
    top_m = int(tune_percentile(ranks, 0.995))
    max_rank = max(ranks)
    hits = np.bincount(np.asarray(ranks) - 1, minlength=max_rank)
    p1, _ = tune_elbow(hits, len(ranks))
    pq_, pl_, pt_, in_p1 = [], [], [], []
    for i in range(nq):
        for t in gt[i]:
            c = list_of.get(int(t), -1)
            if c < 0:
                continue
            pq_.append(i); pl_.append(c); pt_.append(int(t)); in_p1.append(rank_of[i, c] <= min(p1, nl))
    _, _, pr, _, _ = tune_list_stats(q, cent, codebook, offsets, ids, codes, base, pq_, pl_, pt_)
    all_pq = [int(r) for r in pr if r > 0]
    p1_pq = [int(r) for r, f in zip(pr, in_p1) if r > 0 and f]
    limit_k = max(p1_pq) if p1_pq else int(tune_percentile(all_pq, 0.98))
    ratios = []
    for i in range(nq):
        lists = [int(order[i, r]) for r in range(min(p1, nl)) if offsets[order[i, r] + 1] > offsets[order[i, r]]]
        if not lists:
            continue
        _, _, _, _, cut = tune_list_stats(q, cent, codebook, offsets, ids, codes, None, [i] * len(lists), lists,
                                          None, [max(limit_k, 1)] * len(lists))
        far = int(gt[i, k - 1])
        c = list_of.get(far, -1)
        if c < 0:
            continue
        fp, _, _, _, _ = tune_list_stats(q, cent, codebook, offsets, ids, codes, None, [i], [c], [far])
        if fp[0] < 0:
            continue
        mc = np.float32(cut.min())
        if mc > 0:
            ratios.append(np.float32(fp[0] / mc))
    coeff = max(ratios) if ratios else np.float32(2.0)
    return top_m, p1, limit_k, np.float32(coeff)


def graph_search(q, base, graph, k, itopk=64, width=4, max_iter=64, seed=1, nthreads=0):
    """Graph search (own definition, see oracle.cpp): (ids [nq][k], dists [nq][k], steps [nq])."""
    q, base, graph = f32(q), f32(base), i32(graph)
    nq, dim = q.shape
    oid = np.empty((nq, k), np.int32)
    od = np.empty((nq, k), np.float32)
    it = np.empty(nq, np.int32)
    lib.orc_graph_search(_p(q), nq, _p(base), base.shape[0], dim, _p(graph), graph.shape[1], itopk, width, max_iter,
                         k, seed, _p(oid), _p(od), _p(it), nthreads)
    return oid, od, it


def coarse_graph_build(cent, degree, nthreads=0):
    """The centroid graph of the graph coarse mode (fgpu_coarse_graph_build): with F(v) the 2*degree nearest
    other centroids of v (knn_exact, tie rule (distance, id)), row v holds the first degree - degree//2 entries
    of F(v), then the u whose first `degree` entries of F(u) include v, by (rank of v in F(u), u), then the rest
    of F(v), skipping ids already present, up to `degree` ids: int32 [nlist][degree]."""
    cent = f32(cent)
    nl, d2 = cent.shape[0], 2 * degree
    ids, _ = knn_exact(cent, cent, d2 + 1, nthreads)
    fwd = [[int(j) for j in ids[i] if j != i][:d2] for i in range(nl)]
    rev = [[] for _ in range(nl)]
    for u in range(nl):
        for r in range(degree):
            rev[fwd[u][r]].append((r, u))
    nf = degree - degree // 2
    out = np.empty((nl, degree), np.int32)
    for v in range(nl):
        row = []
        for c in fwd[v][:nf] + [u for _, u in sorted(rev[v])] + fwd[v][nf:]:
            if len(row) < degree and c not in row:
                row.append(c)
        out[v] = row
    return out


def coarse_graph(q, cent, graph, nprobe, itopk=32, width=4, max_iter=200, seed=1, prune_ratio=100.0, nthreads=0):
    """The graph coarse mode: graph_search over the centroids, then the prune rule of
    prune_and_count_fused_kernel (gpu_global.cu:43-50) in float32, empty slots pruned:
    (ids uint32 [nq][nprobe], dists float32 [nq][nprobe])."""
    gid, gd, _ = graph_search(q, cent, graph, nprobe, itopk, width, max_iter, seed, nthreads)
    thr = gd[:, :1] * np.float32(prune_ratio)
    ids = gid.view(np.uint32).copy()
    ids[(gid < 0) | (gd > thr)] = 0xFFFFFFFF
    return ids, gd


def graph_bit(node):
    """The visited-bitmap bit of a node id (2^16-bit bitmap, multiplicative hash)."""
    return ((int(node) * 2654435761) & 0xFFFFFFFF) >> 16


def kmeans_assign(x, cent, nthreads=0):
    x, cent = f32(x), f32(cent)
    out = np.empty(x.shape[0], np.int32)
    lib.orc_kmeans_assign(_p(x), x.shape[0], _p(cent), cent.shape[0], x.shape[1], _p(out), nthreads)
    return out


def fixed_shift(maxabs, n):
    return lib.orc_fixed_shift(maxabs, n)


def kmeans_update(x, assign, cent, shift, empty_rule=0):
    x, assign = f32(x), i32(assign)
    cent = f32(cent).copy()
    counts = np.empty(cent.shape[0], np.int32)
    lib.orc_kmeans_update(_p(x), x.shape[0], _p(assign), cent.shape[0], x.shape[1], shift, empty_rule, _p(cent),
                          _p(counts))
    return cent, counts


def kmeans_init_strided(x, k, seed=42):
    x = f32(x)
    out = np.empty((k, x.shape[1]), np.float32)
    rows = np.empty(k, np.int32)
    lib.orc_kmeans_init_strided(_p(x), x.shape[0], x.shape[1], k, seed, _p(out), _p(rows))
    return out, rows


def kmeans_init_pp(x, k, seed, nthreads=0):
    x = f32(x)
    out = np.empty((k, x.shape[1]), np.float32)
    rows = np.empty(k, np.int32)
    lib.orc_kmeans_init_pp(_p(x), x.shape[0], x.shape[1], k, seed, _p(out), _p(rows), nthreads)
    return out, rows


def kmeans_fit(x, k, iters, init_mode=0, seed=42, nthreads=0):
    """run_kmeans_gpu restated: init, then iters x (assign, update); returns (centroids, final assignment)."""
    x = f32(x)
    cent = kmeans_init_strided(x, k, seed)[0] if init_mode == 0 else kmeans_init_pp(x, k, seed, nthreads)[0]
    shift = fixed_shift(float(np.abs(x).max()), x.shape[0])
    for _ in range(iters):
        a = kmeans_assign(x, cent, nthreads)
        cent, _ = kmeans_update(x, a, cent, shift, 0)
    return cent, kmeans_assign(x, cent, nthreads)


def pq_kmeans_fast(data, k, seed, iters):
    data = f32(data)
    out = np.empty((k, data.shape[1]), np.float32)
    if lib.orc_pq_kmeans_fast(_p(data), data.shape[0], data.shape[1], k, seed, iters, _p(out)) != 0:
        raise ValueError("orc_pq_kmeans_fast: n < k")
    return out


def pq_sample(n, sample_size):
    out = np.empty(min(n, sample_size), np.int32)
    lib.orc_pq_sample(n, sample_size, _p(out))
    return out


def pq_train(x, assign, cent, pq_m, sample_size=50000, iters=8, nthreads=0):
    x, assign, cent = f32(x), i32(assign), f32(cent)
    dim = x.shape[1]
    cb = np.empty((pq_m, 256, dim // pq_m), np.float32)
    if lib.orc_pq_train(_p(x), x.shape[0], dim, pq_m, _p(assign), _p(cent), sample_size, iters, _p(cb), nthreads) != 0:
        raise ValueError("orc_pq_train failed")
    return cb


def pq_encode(x, assign, cent, codebook, fma_mode=1, nthreads=0):
    x, assign, cent, codebook = f32(x), i32(assign), f32(cent), f32(codebook)
    pq_m = codebook.shape[0]
    codes = np.empty((x.shape[0], pq_m), np.uint8)
    lib.orc_pq_encode(_p(x), x.shape[0], x.shape[1], pq_m, _p(assign), _p(cent), _p(codebook), fma_mode, _p(codes),
                      nthreads)
    return codes


def build_lists(assign, nlist, codes):
    assign, codes = i32(assign), u8(codes)
    n, m = codes.shape
    offs = np.empty(nlist + 1, np.int32)
    ids = np.empty(n, np.int32)
    lc = np.empty((n, m), np.uint8)
    lib.orc_build_lists(_p(assign), n, nlist, _p(codes), m, _p(offs), _p(ids), _p(lc))
    return offs, ids, lc


def build_ivfpq(x, nlist, pq_m, kmeans_iters=20, init_mode=0, seed=42, pq_iters=8, sample_size=50000, nthreads=0,
                train_rows=0):
    """build_global restated without rebalancing (build_global.cu:21-258).  train_rows > 0: k-means on the
    systematic sample rows floor(j*n/train_rows), then every row assigned to its nearest centroid."""
    n = x.shape[0]
    if 0 < train_rows < n:
        rows = (np.arange(train_rows, dtype=np.int64) * n) // train_rows
        cent, _ = kmeans_fit(np.ascontiguousarray(x[rows]), nlist, kmeans_iters, init_mode, seed, nthreads)
        assign = kmeans_assign(x, cent, nthreads)
    else:
        cent, assign = kmeans_fit(x, nlist, kmeans_iters, init_mode, seed, nthreads)
    cb = pq_train(x, assign, cent, pq_m, sample_size, pq_iters, nthreads)
    codes = pq_encode(x, assign, cent, cb, 1, nthreads)
    offs, ids, lc = build_lists(assign, nlist, codes)
    return offs, ids, lc, cent, cb


def rebalance_buckets(buckets, n_total, nlist, split):
    """The queue-based recursive split of build_global (build_global.cu:62-169), restated.  buckets: the
    initial (rows, centroid) pairs in cluster order; n_total: vectors over all buckets; nlist: the initial
    cluster count (K_CLUSTERS).  avg = n_total / nlist in double; a bucket is final when its size is <= (size_t)
    (2 avg) or < 32; otherwise sub_k = ceil(size / avg), at least 2, at most size / 2 (integer division), and
    split(rows, sub_k) returns the sub_k children (rows, centroid) in child order, whose non-empty ones go to the
    back of the queue.  Empty initial buckets are dropped.  Returns (final buckets in order, split count)."""
    avg = float(n_total) / float(nlist)
    thr = int(avg * 2)
    queue = collections.deque((r, c) for r, c in buckets if len(r) > 0)
    final, splits = [], 0
    while queue:
        rows, c = queue.popleft()
        sz = len(rows)
        if sz <= thr or sz < 32:
            final.append((rows, c))
            continue
        splits += 1
        sub_k = int(math.ceil(sz / avg))
        sub_k = max(sub_k, 2)
        sub_k = min(sub_k, sz // 2)
        for ch_rows, ch_c in split(rows, sub_k):
            if len(ch_rows) > 0:
                queue.append((ch_rows, ch_c))
    return final, splits


def build_global(x, nlist, pq_m, kmeans_iters=20, pq_iters=8, sample_size=50000, init_mode=0, seed=42,
                 rebalance=True, nthreads=0):
    """build_global restated (build_global.cu:21-258): k-means over every row, assignment, the recursive split
    (rebalance_buckets, each split a 15-iteration k-means of the bucket's rows with the same initialisation and
    seed, then their exact assignment; build_global.cu:112-142), PQ training on the final lists, device-form
    encoding, lists in final order with each list's rows ascending.  Without rebalancing every initial list stays,
    empty ones included.  Returns (offsets, ids, codes, centroids, codebook, split count)."""
    x = f32(x)
    n = x.shape[0]
    cent, a0 = kmeans_fit(x, nlist, kmeans_iters, init_mode, seed, nthreads)
    buckets = [(np.nonzero(a0 == c)[0].astype(np.int32), cent[c]) for c in range(nlist)]

    def split(rows, sub_k):
        sub = np.ascontiguousarray(x[rows])
        sc, _ = kmeans_fit(sub, sub_k, 15, init_mode, seed, nthreads)
        la = kmeans_assign(sub, sc, nthreads)
        return [(rows[la == j], sc[j]) for j in range(sub_k)]

    final, splits = rebalance_buckets(buckets, n, nlist, split) if rebalance else (buckets, 0)
    L = len(final)
    assign = np.empty(n, np.int32)
    for c, (rows, _) in enumerate(final):
        assign[rows] = c
    fc = np.ascontiguousarray(np.stack([c for _, c in final]).astype(np.float32))
    cb = pq_train(x, assign, fc, pq_m, sample_size, pq_iters, nthreads)
    codes = pq_encode(x, assign, fc, cb, 1, nthreads)
    offs, ids, lc = build_lists(assign, L, codes)
    return offs, ids, lc, fc, cb, splits


# --------------------------------------------------------------------------- the reference's own code
def ref_lib():
    """The reference's pq_utils.h/utils.h compiled from /root/reference (None if not built)."""
    if not os.path.exists(REF_SO):
        return None
    l = ctypes.CDLL(REF_SO)
    l.ref_run_kmeans_pq_fast.argtypes = [_vp, _i32, _i32, _i32, _i32, _i32, _vp]
    l.ref_train_residual_pq_codebooks.argtypes = [_vp, _i32, _vp, _vp, _i32, _i32, _i32, _vp]
    l.ref_encode_residuals_to_pq.argtypes = [_vp, _i32, _vp, _vp, _i32, _vp, _vp]
    l.ref_read_fvecs.argtypes = [_c.c_char_p, _i32, _c.POINTER(_c.POINTER(_f32))]
    l.ref_read_fvecs.restype = _i32
    l.ref_read_ivecs.argtypes = [_c.c_char_p, _c.POINTER(_i32), _c.POINTER(_c.POINTER(_i32))]
    l.ref_read_ivecs.restype = _i32
    l.ref_free_f.argtypes = [_c.POINTER(_f32)]
    l.ref_free_i.argtypes = [_c.POINTER(_i32)]
    return l
