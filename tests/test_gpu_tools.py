"""The command-line tools on the GPU: build_global writes the same index files
as the library build and, with its recursive rebalancing (build_global.cu:62-169),
the same bytes as the oracle's statement of it; search_pipeline returns the
oracle's ids for its per-batch path and the reference's recall figures
(search_pipeline.cu:531-557, 636-645)."""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no HIP device", allow_module_level=True)

import fusiongpu_amd as fg  # noqa: E402
import oracle  # noqa: E402

BIN = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "fusiongpu_amd", "_lib", "bin")


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _run(*args, cwd):
    r = subprocess.run([os.path.join(BIN, args[0]), *map(str, args[1:])], capture_output=True, text=True,
                       timeout=120, cwd=cwd)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return r.stdout


def _write_ivecs(path, ids):
    ids = np.ascontiguousarray(ids, np.int32)
    rows = np.concatenate([np.full((ids.shape[0], 1), ids.shape[1], np.int32), ids], 1)
    rows.tofile(path)


def _read_ivecs(path):
    a = np.fromfile(path, np.int32)
    k = a[0]
    return a.reshape(-1, k + 1)[:, 1:]


def _build(tmp_path, x, extra):
    res = tmp_path / "res"
    res.mkdir(exist_ok=True)
    fg.write_fvecs(tmp_path / "base.fvecs", x)
    out = _run("build_global", tmp_path / "base.fvecs", "--res", res, *extra, cwd=tmp_path)
    return res, out


def test_build_global_matches_library_build(tmp_path):
    _say("build_global --no-rebalance vs library build")
    x = oracle.gen_gmm(20000, 128, 32, seed=3, sig_lo=0.1)
    res, _ = _build(tmp_path, x, ["--nlist", 64, "--iters", 5, "--pq_iters", 3, "--sample", 5000, "--no-rebalance"])
    offs, ids, codes, cent = fg.read_ivf_data(res / "ivf_data.bin", 32, 128)
    cb = np.fromfile(res / "global_pq_codebook.bin", np.float32).reshape(32, 256, 4)
    want = fg.build_ivfpq(torch.from_numpy(x).cuda(), 64, 32, kmeans_iters=5, init_mode=0, seed=42, pq_iters=3,
                          sample_size=5000)
    for g, w, name in zip((offs, ids, codes, cent, cb), want, ["offsets", "ids", "codes", "centroids", "codebook"]):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8)), name
    csv = np.loadtxt(tmp_path / "cluster_distribution.csv", delimiter=",", skiprows=1, dtype=np.int64)
    assert np.array_equal(csv[:, 1], np.diff(offs))


def test_build_global_rebalances_oversized_lists(tmp_path):
    _say("build_global rebalancing")
    x = oracle.gen_gmm(30000, 128, 6, seed=4, sig_lo=0.05, sig_hi=0.3)
    res, out = _build(tmp_path, x, ["--nlist", 64, "--iters", 4, "--pq_iters", 2, "--sample", 3000])
    m = re.search(r"Cluster Count: 64 -> (\d+)", out)
    assert m and "Split Ops" in out
    offs, ids, codes, cent = fg.read_ivf_data(res / "ivf_data.bin", 32, 128)
    L = int(m.group(1))
    # byte for byte the oracle's statement of build_global with its queue (build_global.cu:21-258)
    cb = np.fromfile(res / "global_pq_codebook.bin", np.float32).reshape(32, 256, 4)
    want = oracle.build_global(x, 64, 32, kmeans_iters=4, pq_iters=2, sample_size=3000)
    for g, w, name in zip((offs, ids, codes, cent, cb), want, ["offsets", "ids", "codes", "centroids", "codebook"]):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8)), name
    assert f"Split Ops: {want[5]}" in out
    assert offs.shape[0] == L + 1 and offs[0] == 0 and offs[-1] == 30000 and np.all(np.diff(offs) > 0)
    assert np.array_equal(np.sort(ids), np.arange(30000))
    sizes = np.diff(offs)
    thr = int(30000 / 64 * 2)
    assert np.all((sizes <= thr) | (sizes < 32)), sizes.max()
    # the codes are the device-form encoding of each vector against its list's centroid
    cb = np.fromfile(res / "global_pq_codebook.bin", np.float32).reshape(32, 256, 4)
    assign = np.empty(30000, np.int32)
    assign[ids] = np.repeat(np.arange(L, dtype=np.int32), sizes)
    assert np.array_equal(codes, oracle.pq_encode(x, assign, cent, cb, fma_mode=1)[ids])
    idx = fg.Index.load(res / "ivf_data.bin", res / "global_pq_codebook.bin", 128, 32)
    assert idx.nlist == L
    idx.close()


def test_search_pipeline_matches_library_path(tmp_path):
    _say("search_pipeline vs library path")
    x = oracle.gen_gmm(20000, 128, 32, seed=5, sig_lo=0.1)
    q = oracle.gen_gmm(300, 128, 32, seed=5, set=1, sig_lo=0.1)
    res, _ = _build(tmp_path, x, ["--nlist", 64, "--iters", 5, "--pq_iters", 3, "--sample", 5000, "--no-rebalance"])
    fg.write_fvecs(tmp_path / "q.fvecs", q)
    gt, _ = oracle.knn_exact(q, x, 20)
    _write_ivecs(tmp_path / "gt.ivecs", gt)
    # batches of 64 over 3 streams: five batches, so the collector thread hands contexts back for reuse
    out = _run("search_pipeline", tmp_path / "base.fvecs", tmp_path / "q.fvecs", tmp_path / "gt.ivecs", "-b", 64,
               "-m", 16, "-r", 500, "-k", 10, "--p1_lists", 4, "--limit_k", 30, "-s", 3, "--res", res, "--out",
               tmp_path / "out.ivecs", cwd=tmp_path)
    assert re.search(r"Total time: [\d.]+ ms, QPS: [\d.e+]+", out)
    assert re.search(r"batch count:\s+5\b", out), out
    got = _read_ivecs(tmp_path / "out.ivecs")
    # the oracle's per-batch path: exact coarse, two-phase scan, early-stopping rerank
    offs, ids, codes, cent = fg.read_ivf_data(res / "ivf_data.bin", 32, 128)
    cb = np.fromfile(res / "global_pq_codebook.bin", np.float32).reshape(32, 256, 4)
    probes, _ = oracle.coarse(q, cent, 16, 100.0)
    tid, _, tcnt, _, _, pre = oracle.search_two_phase(q, cent, cb, offs, ids, codes, probes, 4, 30, 1.0, 500,
                                                      want_pre_cut=True)
    want, _, _ = oracle.rerank(q, x, tid, tcnt, 10, 128, 0.1, 2)
    assert np.array_equal(got, want)
    # the batch-logic table (search_pipeline.cu:286-306): per-batch averages over the five batches of the
    # probed lists' sizes and of the candidates before the rerank_m cut, and the reduction rate
    assert "GPU Batch Logic Fine-grained Breakdown" in out
    amax = int(oracle.probe_counts(probes, offs).astype(np.int64).sum()) // 5
    areal = int(pre.astype(np.int64).sum()) // 5
    assert int(re.search(r"\[Allocated\] Max Potential Candidates: (\d+)", out).group(1)) == amax
    assert int(re.search(r"\[Actual\]\s+Filtered Real Candidates: (\d+)", out).group(1)) == areal
    rate = float(re.search(r"Pruning Reduction Rate: ([\d.]+) %", out).group(1))
    assert abs(rate - 100.0 * (1.0 - areal / amax)) <= 0.051 and areal < amax
    # the reference's recall: whole gt row as the hit set, repeated ids once, hits / (nq * k)
    m = re.search(r"Recall@1: ([\d.]+)%, Recall@10: ([\d.]+)%", out)
    assert m
    for k, printed in ((1, float(m.group(1))), (10, float(m.group(2)))):
        hits = sum(len(set(got[i, :k]) & set(gt[i])) for i in range(q.shape[0]))
        assert abs(100.0 * hits / (q.shape[0] * k) - printed) < 1e-3
    # the full batches replayed HIP graphs (captured by each context's warm-up batch, then replayed for the
    # timed batches: one context replays twice); the same run as separate launches gives the same ids and
    # the per-stage table
    assert re.search(r"Graph replay:\s+[\d.]+ ms a batch, H2D to D2H \(4 batches\)", out), out
    out2 = _run("search_pipeline", tmp_path / "base.fvecs", tmp_path / "q.fvecs", "-b", 64, "-m", 16, "-r", 500, "-k",
                10, "--p1_lists", 4, "--limit_k", 30, "-s", 3, "--res", res, "--graphs", "off", "--out",
                tmp_path / "out2.ivecs", cwd=tmp_path)
    assert np.array_equal(_read_ivecs(tmp_path / "out2.ivecs"), want)
    assert "Graph replay" not in out2 and re.search(r"Sum of stages:\s+[\d.]+ ms", out2), out2
    assert int(re.search(r"\[Actual\]\s+Filtered Real Candidates: (\d+)", out2).group(1)) == areal


def test_search_pipeline_graph_coarse_matches_library_path(tmp_path):
    """--coarse graph: the centroid kNN graph (degree 8) walked with the
    reference's CAGRA parameters (itopk max(32, top_m), width 4, 200 steps)."""
    _say("search_pipeline --coarse graph vs library path")
    x = oracle.gen_gmm(20000, 128, 32, seed=6, sig_lo=0.1)
    q = oracle.gen_gmm(300, 128, 32, seed=6, set=1, sig_lo=0.1)
    res, _ = _build(tmp_path, x, ["--nlist", 256, "--iters", 5, "--pq_iters", 3, "--sample", 5000, "--no-rebalance"])
    fg.write_fvecs(tmp_path / "q.fvecs", q)
    out = _run("search_pipeline", tmp_path / "base.fvecs", tmp_path / "q.fvecs", "-b", 100, "-m", 24, "-r", 400,
               "-k", 10, "--p1_lists", 6, "--limit_k", 20, "-s", 2, "--res", res, "--coarse", "graph", "--out",
               tmp_path / "out.ivecs", cwd=tmp_path)
    assert "centroid graph: 256 nodes, degree 8, itopk 32" in out
    got = _read_ivecs(tmp_path / "out.ivecs")
    # the oracle: its centroid graph and walk, then the same two-phase scan and rerank
    offs, ids, codes, cent = fg.read_ivf_data(res / "ivf_data.bin", 32, 128)
    cb = np.fromfile(res / "global_pq_codebook.bin", np.float32).reshape(32, 256, 4)
    g = oracle.coarse_graph_build(cent, 8)
    probes, _ = oracle.coarse_graph(q, cent, g, 24, itopk=32, width=4, max_iter=200, seed=1, prune_ratio=100.0)
    tid, _, tcnt, _, _ = oracle.search_two_phase(q, cent, cb, offs, ids, codes, probes, 6, 20, 1.0, 400)
    want, _, _ = oracle.rerank(q, x, tid, tcnt, 10, 128, 0.1, 2)
    assert np.array_equal(got, want)


def test_build_global_elbow_sweep(tmp_path):
    _say("build_global --elbow")
    x = oracle.gen_gmm(12000, 128, 24, seed=6, sig_lo=0.1)
    res, out = _build(tmp_path, x, ["--elbow", "16,32,64", "--train_rows", 6000, "--iters", 3, "--pq_iters", 2,
                                    "--sample", 3000, "--no-rebalance", "--init", "pp"])
    sse = [float(v) for v in re.findall(r"Elbow: nlist \d+ SSE ([\d.e+]+)", out)]
    chosen = int(re.search(r"Elbow: chosen nlist (\d+)", out).group(1))
    assert len(sse) == 3 and sse[0] > sse[1] > sse[2]
    # the SSE of each list count: the oracle's k-means of the training sample
    # (run_kmeans_gpu restated), then the oracle's exact distance of every
    # sample row to its nearest centroid, summed
    rows = (np.arange(6000, dtype=np.int64) * 12000) // 6000
    tr = np.ascontiguousarray(x[rows])
    for L, printed in zip((16, 32, 64), sse):
        oc, _ = oracle.kmeans_fit(tr, L, 3, init_mode=1, seed=42)
        _, od = oracle.coarse(tr, oc, 1, prune_ratio=np.inf)
        osse = float(od[:, 0].astype(np.float64).sum())
        assert abs(osse - printed) <= 1e-5 * printed  # the tool prints six significant digits
    xn = np.log2([16, 32, 64]) - 4.0
    xn /= xn[-1]
    yn = (np.array(sse) - sse[-1]) / (sse[0] - sse[-1])
    assert chosen == [16, 32, 64][int(np.argmax((1 - xn) - yn))]
    offs, _, _, _ = fg.read_ivf_data(res / "ivf_data.bin", 32, 128)
    assert offs.shape[0] == chosen + 1
