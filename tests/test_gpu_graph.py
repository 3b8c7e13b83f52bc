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
