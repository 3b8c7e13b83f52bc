"""The reference-signature layer (include/fusiongpu_compat.hpp) on the GPU,
through tests/compat_driver, which calls it the way the reference's callers
do (search_pipeline.cu:311-372, build_global.cu:41-57 and 202-220).  Every
output is compared with the oracle, bit for bit, at the reference's default
search parameters (rerank_m 10000, p1_lists 12, limit_k 50, mini-batch 128,
eps 0.1, beta 2)."""
import os
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

DRIVER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_bin", "compat_driver")


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _run(args):
    assert os.path.exists(DRIVER), "tests/_bin/compat_driver is not built (make -C tests)"
    r = subprocess.run([DRIVER] + [str(a) for a in args], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr
    return r.stdout


@pytest.mark.parametrize("rerank_m", [10000, 100])
def test_batch_logic_and_rerank_with_reference_defaults(tmp_path, rerank_m):
    """The reference's defaults (rerank_m 10000), and rerank_m 100, where
    the cut drops candidates: d_atomic keeps each query's count before the cut
    (query_atomic_counters, gpu_global.cu:349, 493-526), d_stable_cnt and
    d_finished the rerank's final state (gpu_global.cu:603-609, 653-662)."""
    _say(f"compat search: load_ivf_index_to_gpu, run_gpu_batch_logic, run_gpu_rerank (rerank_m {rerank_m})")
    rng = np.random.default_rng(5151)
    dim, m, nlist, n, nq = 128, 32, 64, 60000, 300
    top_m, p1, limit_k, coeff, k, mb, eps, beta, prune = 20, 12, 50, 1.0, 10, 128, 0.1, 2, 1.3
    assign = rng.integers(0, nlist, n).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = (rng.standard_normal((nlist, dim)) * 0.7).astype(np.float32)
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    base = (rng.standard_normal((n, dim)) * 0.7).astype(np.float32)
    q = (rng.standard_normal((nq, dim)) * 0.7).astype(np.float32)
    res = tmp_path / "res"
    res.mkdir()
    fg.write_ivf_data(res / "ivf_data.bin", offs, ids, lc, cent)
    cb.tofile(res / "global_pq_codebook.bin")
    fg.write_fvecs(tmp_path / "q.fvecs", q)
    fg.write_fvecs(tmp_path / "base.fvecs", base)
    probes, pdist = oracle.coarse(q, cent, top_m, prune_ratio=np.inf)  # unpruned; the layer prunes in place
    probes.astype(np.uint32).tofile(tmp_path / "probes.u32")
    pdist.astype(np.float32).tofile(tmp_path / "pdist.f32")
    out = tmp_path / "out"
    out.mkdir()
    _run(["search", res, tmp_path / "q.fvecs", tmp_path / "base.fvecs", tmp_path / "probes.u32",
          tmp_path / "pdist.f32", out, top_m, p1, limit_k, coeff, rerank_m, k, mb, eps, beta, prune, 128])
    rd = lambda name, dt: np.fromfile(out / name, dt)  # noqa: E731
    # prune in place (prune_and_count_fused_kernel): distance > first distance * ratio, in float32
    want = probes.astype(np.uint32).copy()
    want[pdist > pdist[:, :1] * np.float32(prune)] = 0xFFFFFFFF
    assert (want == 0xFFFFFFFF).any() and (want != 0xFFFFFFFF).all(axis=1).any()
    got = rd("pruned.u32", np.uint32).reshape(nq, top_m)
    assert np.array_equal(got, want)
    assert np.array_equal(rd("counts.i32", np.int32), oracle.probe_counts(want, offs))
    oid, od, ocnt, ocut, othr, opre = oracle.search_two_phase(q, cent, cb, offs, ids, lc, want, p1, limit_k, coeff,
                                                              rerank_m, want_pre_cut=True)
    assert np.array_equal(rd("top_counts.i32", np.int32), ocnt)
    assert np.array_equal(rd("atomic.i32", np.int32), opre)
    if rerank_m < 1000:
        assert (opre > ocnt).any()          # the cut dropped candidates: d_atomic is not the kept count
    assert np.array_equal(rd("top_ids.i32", np.int32).reshape(nq, rerank_m), oid)
    assert np.array_equal(_bits(rd("top_dists.f32", np.float32).reshape(nq, rerank_m)), _bits(od))
    assert np.array_equal(_bits(rd("cutoffs.f32", np.float32).reshape(nq, p1)), _bits(ocut))
    assert np.array_equal(_bits(rd("thresholds.f32", np.float32)), _bits(othr))
    fid, fdist, _, ostab, ofin = oracle.rerank(q, base, oid, ocnt, k, mb, eps, beta, want_state=True)
    assert np.array_equal(rd("final_ids.i32", np.int32).reshape(nq, k), fid)
    assert np.array_equal(_bits(rd("final_dists.f32", np.float32).reshape(nq, k)), _bits(fdist))
    assert np.array_equal(rd("stable.i32", np.int32), ostab)
    assert np.array_equal(rd("finished.u8", np.uint8), ofin)


def test_build_functions_match_the_oracle(tmp_path):
    _say("compat build: run_kmeans_gpu, assignments, train_residual_pq_codebooks, both encodings")
    n, k, iters, sample, pq_iters = 20000, 64, 8, 5000, 5
    x = fg.gen_gmm(n, 128, 40, seed=9, sig_lo=0.1)
    fg.write_fvecs(tmp_path / "x.fvecs", x)
    out = tmp_path / "out"
    out.mkdir()
    _run(["build", tmp_path / "x.fvecs", k, iters, sample, pq_iters, out])
    rd = lambda name, dt: np.fromfile(out / name, dt)  # noqa: E731
    ocent, oasg = oracle.kmeans_fit(x, k, iters, init_mode=0, seed=42)
    cent = rd("centroids.f32", np.float32).reshape(k, 128)
    assert np.array_equal(_bits(cent), _bits(ocent))
    asg = rd("assign.i32", np.int32)
    assert np.array_equal(asg, oracle.kmeans_assign(x, cent))
    ocb = oracle.pq_train(x, asg, cent, 32, sample_size=sample, iters=pq_iters)
    cb = rd("codebook.f32", np.float32).reshape(32, 256, 4)
    assert np.array_equal(_bits(cb), _bits(ocb))
    dev = rd("codes_dev.u8", np.uint8).reshape(n, 32)
    host = rd("codes_host.u8", np.uint8).reshape(n, 32)
    assert np.array_equal(dev, oracle.pq_encode(x, asg, cent, cb, fma_mode=1))
    assert np.array_equal(host, oracle.pq_encode(x, asg, cent, cb, fma_mode=0))
