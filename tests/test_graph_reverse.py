"""fgpu_graph_add_reverse on the CPU: CAGRA's reverse-edge step over host
arrays, against a direct statement of the rule on small graphs (row v: its
nearest degree - degree / 2 forward edges, then the rows u whose first
`degree` forward edges hold v, by (rank of v there, u), then the rest of its
forward list; no repeats, no self edges, -1 padding)."""
import numpy as np
import pytest

import fusiongpu_amd as fg


def _direct(fwd, degree):
    n, width = fwd.shape
    rev = [[] for _ in range(n)]
    for u in range(n):
        for r in range(degree):
            v = int(fwd[u, r])
            if 0 <= v < n and v != u:
                rev[v].append((r, u))
    out = np.full((n, degree), -1, np.int32)
    nf = degree - degree // 2
    for v in range(n):
        row = []
        cands = [int(x) for x in fwd[v, :nf]] + [u for _, u in sorted(rev[v])] + [int(x) for x in fwd[v, nf:]]
        for c in cands:
            if 0 <= c < n and c != v and c not in row and len(row) < degree:
                row.append(c)
        out[v, :len(row)] = row
    return out


@pytest.mark.parametrize("n,width,degree,seed", [(50, 8, 4, 1), (200, 16, 8, 2), (300, 12, 12, 3), (7, 6, 3, 4),
                                                 (5000, 16, 8, 5)])
def test_graph_add_reverse_matches_the_rule(n, width, degree, seed):
    rng = np.random.default_rng(seed)
    fwd = rng.integers(-1, n, (n, width)).astype(np.int32)
    fwd[::7, 0] = np.arange(0, n, 7)            # self edges are dropped
    fwd[3, :] = -1                              # a row with no forward edges
    fwd[5, 1] = n + 3                           # out-of-range ids are dropped
    got = fg.graph_add_reverse(fwd, degree, nthreads=3)
    assert np.array_equal(got, _direct(fwd, degree))


def test_graph_add_reverse_rejects_bad_sizes():
    with pytest.raises(fg.FgpuError):
        fg.graph_add_reverse(np.zeros((4, 2), np.int32), 3)
