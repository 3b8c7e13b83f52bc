"""The BASELINE workloads C1-C5 as data: seeded synthetic inputs of each
configuration and the in-run construction of the C5 graph.

No reference counterpart: the reference reads its inputs from .fvecs files
(utils.h:22-48).  The generators are fgpu_gen_gmm (counter-based splitmix64 +
Box-Muller in double), so every host produces the same vectors; the seeds are
fixed here, and bench.py and the tests both take their inputs from this module.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import gen_gmm


@dataclass(frozen=True)
class Config:
    name: str
    n: int              # base vectors
    dim: int
    ncomp: int          # mixture components
    sig_lo: float
    sig_hi: float
    seed: int
    nq: int
    nlist: int
    pq_m: int
    nprobe: int
    k: int
    train_rows: int = 0   # k-means on the systematic sample of this many rows (0 = all)
    kmeans_iters: int = 20
    pq_iters: int = 15


C1 = Config("c1", 100_000, 128, 64, 0.1, 0.1, 2023, 1000, 256, 16, 16, 10)
C2 = Config("c2", 1_000_000, 128, 256, 0.08, 0.08, 2024, 10_000, 1024, 32, 32, 10)
C3 = Config("c3", 10_000_000, 96, 1024, 0.05, 0.15, 2025, 10_000, 4096, 48, 64, 100, train_rows=1_000_000)
C4 = Config("c4", 10_000_000, 128, 1024, 0.05, 0.15, 2027, 0, 4096, 32, 0, 0, train_rows=1_000_000)
C5 = Config("c5", 5_000_000, 128, 256, 0.05, 0.15, 2026, 10_000, 2048, 32, 8, 10, train_rows=1_000_000,
            kmeans_iters=10, pq_iters=8)

# C3's two-phase and rerank parameters: the reference's defaults for p1_lists,
# limit_k, threshold_coeff, mini_batch, eps, beta (defs.h:18-23; search_pipeline.cu:562-569)
# with the config's compaction to the top 1000 and k = 100.
C3_SEARCH = dict(p1_lists=12, limit_k=50, threshold_coeff=1.0, rerank_m=1000, mini_batch=128, eps=0.1, beta=2)
# C5's graph search: fixed out-degree 32, itopk 64, width 4, at most 64 steps.
C5_GRAPH = dict(degree=32, itopk=64, width=4, max_iter=64, random_edges=8)


def base(cfg: Config, n: int | None = None) -> np.ndarray:
    """The base vectors of a configuration (set 0), float32 [n][dim]."""
    return gen_gmm(cfg.n if n is None else n, cfg.dim, cfg.ncomp, seed=cfg.seed, set=0, sig_lo=cfg.sig_lo,
                   sig_hi=cfg.sig_hi)


def queries(cfg: Config, nq: int | None = None) -> np.ndarray:
    """The queries of a configuration (set 1, the same mixture), float32 [nq][dim]."""
    return gen_gmm(cfg.nq if nq is None else nq, cfg.dim, cfg.ncomp, seed=cfg.seed, set=1, sig_lo=cfg.sig_lo,
                   sig_hi=cfg.sig_hi)


def build_index(cfg: Config, dx, seed: int = 42):
    """The configuration's IVF-PQ index built on the GPU from device rows dx
    (k-means++ seeding, Lloyd iterations, PQ training on a 50k sample,
    encoding): host arrays (offsets, ids, codes, centroids, codebook)."""
    from . import build_ivfpq  # noqa: PLC0415
    return build_ivfpq(dx, cfg.nlist, cfg.pq_m, kmeans_iters=cfg.kmeans_iters, init_mode=1, seed=seed,
                       pq_iters=cfg.pq_iters, sample_size=50000,
                       train_rows=min(cfg.train_rows, dx.shape[0]) if cfg.train_rows else 0)


def knn_graph(dx, degree: int = 32, random_edges: int = 4, nlist: int = 2048, pq_m: int = 32, batch: int = 1 << 18,
              reverse: bool = True):
    """C5's fixed out-degree graph over the device rows dx, int32 [n][degree]
    on the device.  Each row's forward candidates are its nearest other rows
    found by this library's IVF-PQ search (nprobe 8, ADC top-64, then the
    exact top `width` + 1 of those 64 by rerank with eps < 0, so every
    candidate is evaluated), self removed: width = degree, or with `reverse`
    min(2 degree, 63), and then CAGRA's reverse-edge step
    (graph_add_reverse: the nearest half of the forward edges, the reverse
    edges by rank, the rest of the forward list).  The last `random_edges`
    slots are then replaced by seeded long-range edges (a counter-based hash
    of (row, slot)).  A kNN graph over a well-separated mixture has no edges
    between components; the long-range edges let a walk from random seeds
    reach the query's component, and the reverse edges reach the nodes that
    no forward list names."""
    import torch  # noqa: PLC0415

    from . import Index, graph_add_reverse, rerank  # noqa: PLC0415
    n, dim = dx.shape
    width = min(2 * degree, 63) if reverse else degree
    gcfg = Config("c5-graph", n, dim, 0, 0.0, 0.0, 0, 0, nlist, pq_m, 8, 64, train_rows=min(n, 1_000_000),
                  kmeans_iters=10, pq_iters=8)
    offs, ids, codes, cent, cb = build_index(gcfg, dx, seed=7)
    idx = Index.from_arrays(dim, pq_m, offs, ids, codes, cent, cb)
    fwd = torch.empty((n, width), dtype=torch.int32, device=dx.device)
    sws = torch.empty(idx.search_workspace_bytes(min(batch, n), 8), dtype=torch.uint8, device=dx.device)
    cnt64 = torch.full((batch,), 64, dtype=torch.int32, device=dx.device)
    for b0 in range(0, n, batch):
        nb = min(batch, n - b0)
        aid, _ = idx.search(dx[b0:b0 + nb], 8, 64, workspace=sws)
        gid, _, _ = rerank(dx[b0:b0 + nb], dx, aid, cnt64[:nb], width + 1, 64, -1.0, 2)
        rows = torch.arange(b0, b0 + nb, device=dx.device, dtype=torch.int32)[:, None]
        drop = (gid == rows) | (gid < 0)
        order = torch.argsort(drop.to(torch.int8), dim=1, stable=True)[:, :width]
        fwd[b0:b0 + nb] = torch.where(torch.gather(drop, 1, order), -1, torch.gather(gid, 1, order))
    idx.check()
    idx.close()
    if reverse:
        graph = torch.from_numpy(graph_add_reverse(fwd.cpu().numpy(), degree)).to(dx.device)
    else:
        graph = fwd
    del fwd
    if random_edges > 0:
        r = torch.arange(n, device=dx.device, dtype=torch.int64)[:, None] * 1000003 + torch.arange(
            random_edges, device=dx.device, dtype=torch.int64)[None, :] * 7919 + 12345
        r = (r * 6364136223846793005 + 1442695040888963407) & ((1 << 62) - 1)
        graph[:, degree - random_edges:] = ((r >> 17) % n).to(torch.int32)
    return graph
