"""Pins the oracle's graph search (A19).

The reference delegates this to cuVS CAGRA (cagra_adapter.cuh:38-68), which
is not in the repository, so parity with the reference is unpinned and the
oracle states its own definition (oracle.cpp, orc_graph_search).  These tests
fix that definition from outside: on a complete graph it must equal brute-force
exact kNN (orc_knn_exact, pinned by brute force); on a path graph it must walk
to the exact answer with the tie rule; with max_iter = 0 it must return the
best of its 64 seed nodes; and a planted visited-bitmap collision must hide
the node it collides with.
"""
import numpy as np
import pytest

import oracle

FMAX = np.finfo(np.float32).max
M64 = (1 << 64) - 1


def _mix64(z):
    z = (z + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _seeds(seed, q, n):
    return [(_mix64(seed ^ _mix64((q << 20) | j))) % n for j in range(64)]


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("n,k", [(33, 10), (20, 20), (30, 1)])
def test_complete_graph_is_exact_knn(n, k):
    rng = np.random.default_rng(n + k)
    base = rng.standard_normal((n, 24)).astype(np.float32)
    base[5] = base[2]                     # an exact distance tie: the lower id first
    q = rng.standard_normal((6, 24)).astype(np.float32)
    assert len({oracle.graph_bit(i) for i in range(n)}) == n   # no bitmap collisions among the nodes
    graph = np.array([[j for j in range(n) if j != i] + [-1] * (32 - (n - 1)) for i in range(n)], np.int32)
    oid, od, it = oracle.graph_search(q, base, graph, k, itopk=64, width=1, max_iter=64)
    kid, kd = oracle.knn_exact(q, base, k)
    assert np.array_equal(oid, kid) and np.array_equal(_bits(od), _bits(kd))
    assert np.all(it >= 1)


def test_path_graph_walks_to_the_exact_answer():
    n = 2000
    base = np.zeros((n, 4), np.float32)
    base[:, 0] = np.arange(n, dtype=np.float32)
    graph = np.stack([np.arange(n) - 1, np.arange(n) + 1], 1).astype(np.int32)
    graph[n - 1, 1] = -1                  # ids outside [0, n) are skipped
    q = base[[1000, 3]].copy()
    oid, od, it = oracle.graph_search(q, base, graph, 5, itopk=8, width=1, max_iter=5000)
    assert list(oid[0]) == [1000, 999, 1001, 998, 1002]          # ties at distance 1 and 4: lower id first
    assert list(od[0]) == [0.0, 1.0, 1.0, 4.0, 4.0]
    assert list(oid[1]) == [3, 2, 4, 1, 5]
    # the walk stops once every list entry is expanded, long before max_iter
    assert np.all(it < 5000)
    # no steps: the answer is the best of the 64 seeds
    oid0, od0, it0 = oracle.graph_search(q, base, graph, 5, itopk=64, width=1, max_iter=0)
    assert np.all(it0 == 0)
    for i, t in enumerate([1000, 3]):
        s = np.unique(_seeds(1, i, n))
        d = (s.astype(np.float64) - t) ** 2
        order = np.lexsort((s, d))[:5]
        assert list(oid0[i]) == list(s[order])


def test_visited_bitmap_collision_hides_a_node():
    n = 70000
    a = 1234
    b = next(i for i in range(a + 1, n) if oracle.graph_bit(i) == oracle.graph_bit(a))
    c = next(i for i in range(a + 1, n) if oracle.graph_bit(i) not in (oracle.graph_bit(a),)
             and i != b and oracle.graph_bit(i) not in {oracle.graph_bit(s) for s in _seeds(1, 0, n)})
    seeds = set(_seeds(1, 0, n))
    assert not ({a, b, c} & seeds)
    base = np.full((n, 4), 100.0, np.float32)
    base[a, 0] = 1.0                       # second nearest
    base[b, 0] = 0.5                       # nearest, but its bit is a's bit
    base[c, 0] = 0.5
    q = np.zeros((1, 4), np.float32)
    q[0, 1:] = 100.0
    for target, found in ((b, False), (c, True)):
        graph = np.full((n, 2), a, np.int32)   # every node leads to a ...
        graph[a] = target                      # ... and a leads to the target
        graph[target] = target
        oid, od, it = oracle.graph_search(q, base, graph, 2, itopk=64, width=1, max_iter=200)
        assert (oid[0, 0] == target) == found and oid[0, int(found)] == a


@pytest.mark.parametrize("nlist,nprobe,prune", [(33, 10, 100.0), (33, 32, 100.0), (20, 16, 1.3)])
def test_coarse_graph_exhaustive_equals_exact_coarse(nlist, nprobe, prune):
    """The graph coarse mode (the reference's CAGRA-over-centroids step,
    cagra_adapter.cuh:38-68) restated as graph_search over the centroids plus
    the prune rule.  On the complete graph (degree nlist - 1) with
    itopk = 64 >= nlist the first expansion evaluates every centroid, so the
    result must equal the exact coarse quantizer (orc_coarse, pinned by brute
    force) bit for bit, pruned probes included."""
    rng = np.random.default_rng(nlist + nprobe)
    cent = (rng.standard_normal((nlist, 96)) * 0.6).astype(np.float32)
    cent[7] = cent[3]                                   # equal distances: the lower list id first
    graph = np.array([[j for j in range(nlist) if j != i] for i in range(nlist)], np.int32)
    q = (rng.standard_normal((30, 96)) * 0.6).astype(np.float32)
    gid, gd = oracle.coarse_graph(q, cent, graph, nprobe, itopk=64, width=4, max_iter=200, seed=5, prune_ratio=prune)
    eid, ed = oracle.coarse(q, cent, nprobe, prune_ratio=prune)
    assert np.array_equal(gid, eid)
    assert np.array_equal(gd.view(np.uint32), ed.view(np.uint32))
    if prune < 2.0:
        assert np.any(gid == 0xFFFFFFFF)


def test_coarse_graph_build_rule():
    """The centroid graph by brute force: the nearest others in float64 (no
    near-ties in this data) give F(v); forward part, reverse edges by (rank,
    id), then the remaining forward entries."""
    rng = np.random.default_rng(2)
    cent = rng.standard_normal((200, 128)).astype(np.float32)
    cent[50] = cent[10]                                 # a duplicate centroid: its twin comes first
    deg = 6
    g = oracle.coarse_graph_build(cent, deg)
    d = ((cent[:, None, :].astype(np.float64) - cent[None, :, :]) ** 2).sum(-1)
    fwd = [[j for j in np.lexsort((np.arange(200), d[i])) if j != i][:2 * deg] for i in range(200)]
    for v in range(200):
        want = list(fwd[v][:3])
        rev = sorted((fwd[u].index(v), u) for u in range(200) if v in fwd[u][:deg])
        for c in [u for _, u in rev] + fwd[v][3:]:
            if len(want) < deg and c not in want:
                want.append(c)
        assert list(g[v]) == want, v
        assert v not in g[v] and len(set(g[v])) == deg
    assert g[10][0] == 50 and g[50][0] == 10
