"""CPU oracle for parity tests -- TEST INFRASTRUCTURE ONLY.

ctypes wrappers over oracle/liboracle.so (oracle.cpp, the CPU restatement of
the reference's search and build path) and, when built, oracle/_ref/libref.so
(the reference's own pq_utils.h/utils.h compiled from /root/reference).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
package, and only as the checker or the timed CPU baseline.
"""
from __future__ import annotations

import ctypes
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
                                    _f32, _i32, _vp, _vp, _vp, _vp, _vp, _i32]),
    "orc_rerank": (None, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp, _i32]),
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
                     nthreads=0):
    """run_gpu_batch_logic restated: (top_ids [nq][rerank_m], top_dists, counts [nq], cutoffs [nq][p1], thr [nq])."""
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
    lib.orc_search_two_phase(_p(q), nq, dim, codebook.shape[0], _p(cent), _p(codebook), _p(offsets), _p(ids),
                             _p(codes), cent.shape[0], _p(probe_ids), nprobe, p1_lists, limit_k, threshold_coeff,
                             rerank_m, _p(oid), _p(od), _p(cnt), _p(cut), _p(thr), nthreads)
    return oid, od, cnt, cut[:, :p1], thr


def rerank(q, base, cand_ids, counts, k, mb=128, eps=0.1, beta=2, nthreads=0):
    """run_gpu_rerank restated: (ids [nq][k], dists [nq][k], visited [nq])."""
    q, base, cand_ids, counts = f32(q), f32(base), i32(cand_ids), i32(counts)
    nq, dim = q.shape
    rm = cand_ids.shape[1]
    oid = np.empty((nq, k), np.int32)
    od = np.empty((nq, k), np.float32)
    vis = np.empty(nq, np.int32)
    lib.orc_rerank(_p(q), nq, dim, _p(base), base.shape[0], _p(cand_ids), _p(counts), rm, k, mb, eps, beta, _p(oid),
                   _p(od), _p(vis), nthreads)
    return oid, od, vis


def knn_exact(q, base, k, nthreads=0):
    q, base = f32(q), f32(base)
    oid = np.empty((q.shape[0], k), np.int32)
    od = np.empty((q.shape[0], k), np.float32)
    lib.orc_knn_exact(_p(q), q.shape[0], _p(base), base.shape[0], q.shape[1], k, _p(oid), _p(od), nthreads)
    return oid, od


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
