"""Parity at the BASELINE configurations' full sizes: each test builds its
index on the GPU in-test from the configuration's seeded data, runs the HIP
path through the C ABI and compares it with the CPU oracle, bit for bit (ids,
distances, counts, codes, assignments).  Where the oracle would take minutes
the comparison runs on a seeded sample of queries or rows, and the rest of
the output is checked through properties that hold at any size.

Reference call sites of the paths compared: the per-batch search of
SearchPipeline::submit_batch (search_pipeline.cu:341-361) through
run_gpu_batch_logic (gpu_global.cu:679-874) and run_gpu_rerank
(gpu_global.cu:667-673); the index build of build_global (build_global.cu:21-258).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no HIP device", allow_module_level=True)

import fusiongpu_amd as fg  # noqa: E402
import oracle  # noqa: E402
from fusiongpu_amd import workloads as W  # noqa: E402


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _free():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _rows_equal(g, o, what):
    bad = np.nonzero(~np.all(g == o, axis=1))[0]
    assert bad.size == 0, f"{what}: {bad.size} rows differ, first {bad[:5]}: gpu {g[bad[0]]} oracle {o[bad[0]]}"


def test_c2_full_size_every_query():
    """C2 (the north star): 1M x 128, 1024 lists, M=32, all 10k queries in one
    batch, nprobe 32, k 10.  Probes, ids and distances of every query equal the
    oracle's exhaustive search."""
    cfg = W.C2
    _say("c2: generate 1M x 128 + 10k queries, build on the GPU")
    x, q = W.base(cfg), W.queries(cfg)
    dx = torch.from_numpy(x).cuda()
    offs, ids, codes, cent, cb = W.build_index(cfg, dx)
    del dx
    idx = fg.Index.from_arrays(cfg.dim, cfg.pq_m, offs, ids, codes, cent, cb)
    dq = torch.from_numpy(q).cuda()
    _say("c2: GPU coarse + search")
    gp, gpd = idx.coarse_search(dq, cfg.nprobe)
    gid, gd = idx.search(dq, cfg.nprobe, cfg.k)
    gp, gpd, gid, gd = _host(gp).view(np.uint32), _host(gpd), _host(gid), _host(gd)
    assert idx.faults() == 0
    _say("c2: oracle coarse + exhaustive ADC search of all 10k queries")
    op, opd = oracle.coarse(q, cent, cfg.nprobe)
    _rows_equal(gp, op, "c2 probes")
    assert np.array_equal(_bits(gpd), _bits(opd))
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, codes, op, cfg.k)
    _rows_equal(gid, oid, "c2 ids")
    assert np.array_equal(_bits(gd), _bits(od))
    assert (gid >= 0).all()
    idx.close()
    _free()


def test_c3_full_size_sampled_queries():
    """C3: 10M x 96, 4096 lists, M=48, nprobe 64, the two-phase pruned scan
    compacted to the top 1000, exact rerank to k 100.  Every query runs on the
    GPU; 200 seeded queries are compared with the oracle's two-phase search
    (top-1000 ids, distances, counts) and rerank (ids, distances, visited)."""
    cfg, sp = W.C3, W.C3_SEARCH
    _say("c3: generate 10M x 96 + 10k queries, build on the GPU (k-means on a 1M sample)")
    x, q = W.base(cfg), W.queries(cfg)
    dx = torch.from_numpy(x).cuda()
    offs, ids, codes, cent, cb = W.build_index(cfg, dx)
    idx = fg.Index.from_arrays(cfg.dim, cfg.pq_m, offs, ids, codes, cent, cb)
    dq = torch.from_numpy(q).cuda()
    _say("c3: GPU coarse + two-phase + rerank of all 10k queries")
    fid, fd = idx.search_rerank(dq, dx, cfg.nprobe, cfg.k, **sp)
    probes, _ = idx.coarse_search(dq, cfg.nprobe)
    tid, td, tc, cut, thr = idx.two_phase_search(dq, probes, sp["p1_lists"], sp["limit_k"], sp["threshold_coeff"],
                                                 sp["rerank_m"], want_cutoffs=True)
    rid, rd, vis = fg.rerank(dq, dx, tid, tc, cfg.k, sp["mini_batch"], sp["eps"], sp["beta"])
    fid, fd, rid, rd = _host(fid), _host(fd), _host(rid), _host(rd)
    assert np.array_equal(fid, rid) and np.array_equal(_bits(fd), _bits(rd)), "one-call path differs from stages"
    s = np.sort(np.random.default_rng(33).choice(cfg.nq, 200, replace=False))
    qs = q[s]
    _say("c3: oracle coarse + two-phase + rerank of 200 sampled queries")
    op, _ = oracle.coarse(qs, cent, cfg.nprobe)
    _rows_equal(_host(probes).view(np.uint32)[s], op, "c3 probes")
    oid, od, ocnt, ocut, othr = oracle.search_two_phase(qs, cent, cb, offs, ids, codes, op, sp["p1_lists"],
                                                        sp["limit_k"], sp["threshold_coeff"], sp["rerank_m"])
    assert np.array_equal(_host(tc)[s], ocnt)
    _rows_equal(_host(tid)[s], oid, "c3 top-1000 ids")
    assert np.array_equal(_bits(_host(td)[s]), _bits(od))
    assert np.array_equal(_bits(_host(cut)[s]), _bits(ocut))
    assert np.array_equal(_bits(_host(thr)[s]), _bits(othr))
    fid_o, fd_o, vis_o = oracle.rerank(qs, x, oid, ocnt, cfg.k, sp["mini_batch"], sp["eps"], sp["beta"])
    _rows_equal(rid[s], fid_o, "c3 reranked ids")
    assert np.array_equal(_bits(rd[s]), _bits(fd_o))
    assert np.array_equal(_host(vis)[s], vis_o)
    idx.close()
    del dx
    _free()


def test_c4_full_size_build_properties():
    """C4: 10M x 128, k-means++ + 20 Lloyd iterations of 4096 centroids on a
    1M-row sample, every row assigned, PQ M=32 (15 iterations), every row
    encoded.  The lists are a permutation with ascending ids inside each list;
    for 20k seeded rows the list equals the oracle's exact argmin over the
    GPU centroids and the codes equal the oracle's encoding; the codebook
    equals the oracle's PQ training on the same assignment and 50k sample
    (pq_utils.h:77-138); a Lloyd update of the training sample's final
    assignment equals the oracle's fixed-point update.  Then the elbow sweep
    over 1024/2048/4096 lists (tune_parameters.cu:199-456 scores the same
    SSE): each SSE over the 1M-row sample equals the sum of the oracle's exact
    distances from every sample row to its nearest GPU centroid, row by row
    bit for bit, and the knee follows from those SSEs."""
    cfg = W.C4
    _say("c4: generate 10M x 128, build 4096 lists on the GPU")
    x = W.base(cfg)
    dx = torch.from_numpy(x).cuda()
    offs, ids, codes, cent, cb = W.build_index(cfg, dx)
    n = cfg.n
    assert offs[0] == 0 and offs[-1] == n and (np.diff(offs) >= 0).all()
    perm = np.zeros(n, np.int8)
    perm[ids] = 1
    assert perm.all(), "ids are not a permutation of the rows"
    lid = np.repeat(np.arange(cfg.nlist, dtype=np.int32), np.diff(offs))
    inner = np.diff(ids) > 0
    assert inner[np.diff(lid) == 0].all(), "ids not ascending inside a list"
    row_list = np.empty(n, np.int32)
    row_list[ids] = lid
    row_code = np.empty((n, cfg.pq_m), np.uint8)
    row_code[ids] = codes
    s = np.sort(np.random.default_rng(44).choice(n, 20000, replace=False))
    _say("c4: oracle exact assignment + encoding of 20k sampled rows")
    oa = oracle.kmeans_assign(x[s], cent)
    assert np.array_equal(row_list[s], oa)
    oc = oracle.pq_encode(x[s], oa, cent, cb, fma_mode=1)
    assert np.array_equal(row_code[s], oc)
    _say("c4: oracle PQ training on the full assignment (50k sample, 15 iterations)")
    ocb = oracle.pq_train(x, row_list, cent, cfg.pq_m, sample_size=50000, iters=cfg.pq_iters)
    assert np.array_equal(_bits(cb), _bits(ocb))
    # the Lloyd update at the training sample's full size
    _say("c4: one fixed-point Lloyd update of the 1M-row sample against the oracle")
    rows = (np.arange(cfg.train_rows, dtype=np.int64) * n) // cfg.train_rows
    xs = x[rows]
    dxs = torch.from_numpy(xs).cuda()
    asg, _ = fg.l2_topk(dxs, torch.from_numpy(cent).cuda(), 1)
    asg = asg[:, 0].contiguous()
    shift = fg.fixed_shift(float(np.abs(xs).max()), xs.shape[0])
    gc = torch.from_numpy(cent).cuda()
    cnt = fg.kmeans_update(dxs, asg, gc, shift)
    oc2, ocnt2 = oracle.kmeans_update(xs, _host(asg), cent, shift)
    assert np.array_equal(_host(cnt), ocnt2)
    assert np.array_equal(_bits(_host(gc)), _bits(oc2))
    del dx
    _free()
    # the elbow sweep on the training sample
    sse = {}
    for L in (1024, 2048, 4096):
        _say(f"c4: elbow sweep, k-means of {L} lists on the GPU, oracle exact distances of the 1M sample rows")
        c, _ = fg.kmeans_fit(dxs, L, cfg.kmeans_iters, init_mode=1, seed=42, want_assign=False)
        if L == cfg.nlist:
            assert np.array_equal(_bits(_host(c)), _bits(cent)), "the sweep's 4096 lists differ from the build's"
        _, d = fg.l2_topk(dxs, c, 1)
        gsse = float(d.to(torch.float64).sum().item())
        _, od = oracle.coarse(xs, _host(c), 1, prune_ratio=np.inf)
        assert np.array_equal(_bits(_host(d)[:, 0]), _bits(od[:, 0]))
        osse = float(od[:, 0].astype(np.float64).sum())
        assert gsse == osse
        sse[L] = osse
    assert sse[1024] > sse[2048] > sse[4096]
    xn = np.log2([1024, 2048, 4096]) - 10.0
    xn /= xn[-1]
    yv = np.array([sse[1024], sse[2048], sse[4096]])
    yn = (yv - yv[-1]) / (yv[0] - yv[-1])
    knee = [1024, 2048, 4096][int(np.argmax((1 - xn) - yn))]
    _say(f"c4: elbow SSE {sse}, knee at {knee} lists")
    del dxs
    _free()


def test_c5_full_size_graph_search():
    """C5: graph search over 5M x 128 with a fixed out-degree-32 graph, 10k
    queries, itopk 64, width 4, at most 64 steps, k 10.  All queries run on the
    GPU; the first 200 (a query's seed nodes depend on its index) are compared
    with the oracle's statement of the walk: ids, distances and steps."""
    cfg, gp = W.C5, W.C5_GRAPH
    _say("c5: generate 5M x 128 + 10k queries, build the degree-32 graph on the GPU")
    x, q = W.base(cfg), W.queries(cfg)
    dx = torch.from_numpy(x).cuda()
    graph = W.knn_graph(dx, gp["degree"], gp["random_edges"])
    dq = torch.from_numpy(q).cuda()
    _say("c5: GPU graph search of all 10k queries")
    gid, gd, git = fg.graph_search(dq, dx, graph, cfg.k, gp["itopk"], gp["width"], gp["max_iter"], seed=1)
    gid, gd, git = _host(gid), _host(gd), _host(git)
    hg = _host(graph)
    # -1 pads a row whose vector had fewer than degree other candidates; the
    # search skips ids outside [0, n)
    assert ((hg >= -1) & (hg < cfg.n)).all() and (hg >= 0).mean() > 0.99
    ns = 200
    _say("c5: oracle graph walk of the first 200 queries")
    oid, od, oit = oracle.graph_search(q[:ns], x, hg, cfg.k, gp["itopk"], gp["width"], gp["max_iter"], seed=1)
    _rows_equal(gid[:ns], oid, "c5 ids")
    assert np.array_equal(_bits(gd[:ns]), _bits(od))
    assert np.array_equal(git[:ns], oit)
    assert (gid >= 0).all()
    del dx, graph
    _free()
