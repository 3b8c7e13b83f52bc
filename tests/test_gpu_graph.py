"""GPU parity for the graph search (A19): the HIP kernel through the C ABI
against the oracle's statement of the same algorithm, on the same seeded
inputs.  Bar: bit-exact ids, distances and step counts.  (Parity with the
reference's cuVS CAGRA is unpinned: cuVS is not in the reference.)
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


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _knn_graph(x, degree):
    """Exact kNN graph of x (self excluded) from the GPU exact kNN."""
    ids, _ = fg.knn_exact(torch.from_numpy(x).cuda(), torch.from_numpy(x).cuda(), degree + 1)
    ids = _host(ids)
    out = np.empty((x.shape[0], degree), np.int32)
    for i in range(x.shape[0]):
        row = ids[i][ids[i] != i][:degree]
        out[i] = row
    return out


# (n, dim, degree, itopk, width, max_iter, k)
CASES = [(20000, 128, 32, 64, 4, 64, 10), (15000, 96, 16, 32, 8, 40, 32), (8000, 128, 32, 64, 1, 200, 64),
         (40, 96, 8, 16, 2, 10, 5), (5000, 128, 32, 64, 4, 0, 10)]


@pytest.mark.parametrize("n,dim,degree,itopk,width,max_iter,k", CASES)
def test_graph_search_bit_exact(n, dim, degree, itopk, width, max_iter, k):
    _say(f"graph n={n} dim={dim} degree={degree} itopk={itopk} width={width} max_iter={max_iter} k={k}")
    x = oracle.gen_gmm(n, dim, max(4, n // 500), seed=n + dim, sig_lo=0.1)
    q = oracle.gen_gmm(200, dim, max(4, n // 500), seed=n + dim, set=1, sig_lo=0.1)
    graph = _knn_graph(x, degree)
    graph[3, 0] = -5                      # ids outside [0, n) are skipped
    graph[4, 1] = n + 7
    gid, gd, git = fg.graph_search(torch.from_numpy(q).cuda(), torch.from_numpy(x).cuda(),
                                   torch.from_numpy(graph).cuda(), k, itopk, width, max_iter, seed=9)
    oid, od, oit = oracle.graph_search(q, x, graph, k, itopk, width, max_iter, seed=9)
    gid, gd, git = _host(gid), _host(gd), _host(git)
    assert np.array_equal(git, oit), np.nonzero(git != oit)[0][:5]
    bad = np.nonzero(~np.all(gid == oid, axis=1))[0]
    assert bad.size == 0, f"first mismatching queries {bad[:5]}"
    assert np.array_equal(_bits(gd), _bits(od))


def _centroid_index(rng, nlist, dim, m=16):
    """An index whose centroids are the point of the test (lists hold a few random codes)."""
    n = 4 * nlist
    assign = rng.integers(0, nlist, n).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = oracle.gen_gmm(nlist, dim, max(2, nlist // 4), seed=nlist + dim, sig_lo=0.08)
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.1).astype(np.float32)
    return fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb), cent


# (nlist, dim, degree, nprobe, itopk, width, max_iter, prune_ratio)
COARSE_CASES = [(1024, 128, 8, 32, 32, 4, 200, 100.0),   # C2 shape with the reference's search parameters
                (4096, 96, 8, 64, 64, 4, 200, 100.0),    # C3 shape
                (1024, 128, 16, 20, 48, 2, 30, 1.02)]    # a tight prune ratio, few steps


@pytest.mark.parametrize("nlist,dim,degree,nprobe,itopk,width,max_iter,prune", COARSE_CASES)
def test_coarse_graph_bit_exact(nlist, dim, degree, nprobe, itopk, width, max_iter, prune):
    _say(f"coarse graph nlist={nlist} dim={dim} degree={degree} nprobe={nprobe} itopk={itopk} width={width} "
         f"max_iter={max_iter} prune={prune}")
    rng = np.random.default_rng(nlist + degree)
    idx, cent = _centroid_index(rng, nlist, dim)
    g = _host(idx.coarse_graph_build(degree))
    assert np.array_equal(g, oracle.coarse_graph_build(cent, degree))
    q = oracle.gen_gmm(400, dim, max(2, nlist // 4), seed=nlist + dim, set=1, sig_lo=0.08)
    dq, dg = torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda()
    gid, gd = idx.coarse_graph_search(dq, nprobe, dg, itopk, width, max_iter, seed=7, prune_ratio=prune)
    gid, gd = _host(gid).view(np.uint32), _host(gd)
    # two batches, the second starting at query 150, give the one-call result
    a1, _ = idx.coarse_graph_search(dq[:150], nprobe, dg, itopk, width, max_iter, seed=7, prune_ratio=prune)
    a2, _ = idx.coarse_graph_search(dq[150:], nprobe, dg, itopk, width, max_iter, seed=7, prune_ratio=prune,
                                    first_query=150)
    assert np.array_equal(np.concatenate([_host(a1), _host(a2)]).view(np.uint32), gid)
    oid, od = oracle.coarse_graph(q, cent, g, nprobe, itopk, width, max_iter, seed=7, prune_ratio=prune)
    bad = np.nonzero(~np.all(gid == oid, axis=1))[0]
    assert bad.size == 0, f"first mismatching queries {bad[:5]}"
    assert np.array_equal(_bits(gd), _bits(od))
    if prune < 2.0:
        assert np.any(gid == 0xFFFFFFFF)
    # quality against the exact coarse quantizer (reported; the walk is approximate by design)
    eid, _ = oracle.coarse(q, cent, nprobe, prune_ratio=prune)
    hit = np.mean([len(set(a[a != 0xFFFFFFFF]) & set(b[b != 0xFFFFFFFF])) / max(1, np.sum(b != 0xFFFFFFFF))
                   for a, b in zip(gid, eid)])
    _say(f"coarse graph recall of the exact top-{nprobe}: {hit:.4f}")
    assert hit > 0.3
    idx.close()


def test_coarse_graph_exhaustive_equals_coarse_search():
    """Complete graph over 33 centroids, itopk 64: the walk evaluates every
    centroid, so the result equals fgpu_coarse_search bit for bit."""
    _say("coarse graph exhaustive")
    rng = np.random.default_rng(33)
    idx, cent = _centroid_index(rng, 33, 96)
    g = torch.from_numpy(np.array([[j for j in range(33) if j != i] for i in range(33)], np.int32)).cuda()
    q = torch.from_numpy(oracle.gen_gmm(200, 96, 8, seed=4, set=1, sig_lo=0.08)).cuda()
    for prune in (100.0, 1.2):
        gid, gd = idx.coarse_graph_search(q, 16, g, itopk=64, width=4, max_iter=200, seed=3, prune_ratio=prune)
        eid, ed = idx.coarse_search(q, 16, prune_ratio=prune)
        assert np.array_equal(_host(gid), _host(eid))
        assert np.array_equal(_bits(_host(gd)), _bits(_host(ed)))
    idx.close()
