"""GPU parity for the offline tuner (tune_parameters.cu:459-1053): the batched
per-(query, list) statistics kernel against the CPU oracle (bit-exact
distances, ranks and k-th values), and the tune_parameters tool end to end
against the oracle's restatement of the tuner on the same sampled queries."""
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


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("dim,m", [(128, 32), (96, 16), (96, 48), (128, 64)])
def test_tune_list_stats_bit_exact(dim, m):
    _say(f"tune_list_stats dim={dim} m={m}")
    rng = np.random.default_rng(dim + m)
    nlist, n = 24, 12000
    p = rng.random(nlist) + 0.05
    p[4] = 0.0                                   # an empty list
    p[9] *= 30.0                                 # a long list
    assign = rng.choice(nlist, size=n, p=p / p.sum()).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    codes[11] = codes[10]                        # equal PQ distances inside a list
    assign[11] = assign[10]
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = (rng.standard_normal((nlist, dim)) * 0.7).astype(np.float32)
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    base = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((40, dim)).astype(np.float32)
    npairs = 600
    pq = rng.integers(0, 40, npairs).astype(np.int32)
    pl = rng.integers(0, nlist, npairs).astype(np.int32)
    pt = np.empty(npairs, np.int32)
    for j in range(npairs):                      # mostly a member of the list, sometimes not
        lo, hi = offs[pl[j]], offs[pl[j] + 1]
        pt[j] = ids[rng.integers(lo, hi)] if hi > lo and j % 5 else int(rng.integers(-1, n))
    pk = rng.integers(-1, 400, npairs).astype(np.int32)
    pk[:3] = [1, 100000, 0]
    pl[3], pq[4], pl[5] = 4, 40, nlist           # the empty list; a pair outside the inputs (query, list)
    pl[6], pt[6] = 9, ids[offs[9] + 1]           # the long list
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    g = idx.tune_list_stats(torch.from_numpy(q).cuda(), pq, pl, pt, pk, base=torch.from_numpy(base).cuda())
    o = oracle.tune_list_stats(q, cent, cb, offs, ids, lc, base, pq, pl, pt, pk)
    names = ["target_pq", "target_exact", "pq_rank", "exact_rank"]
    for gv, ov, name in zip(g[:4], o[:4], names):
        gv = _host(gv)
        assert np.array_equal(gv.view(np.uint32), np.asarray(ov).view(np.uint32)), name
    sel = pk > 0
    assert np.array_equal(_bits(_host(g[4]))[sel], _bits(o[4])[sel])
    assert _host(g[2])[4] == 0 and _host(g[0])[4] == -1
    # no target and no raw vectors: only the k-th values
    g2 = idx.tune_list_stats(torch.from_numpy(q).cuda(), pq, pl, None, pk)
    assert g2[0] is None and np.array_equal(_bits(_host(g2[4]))[sel], _bits(o[4])[sel])
    idx.close()


def test_tune_parameters_tool_matches_oracle(tmp_path):
    _say("tune_parameters end to end")
    x = oracle.gen_gmm(20000, 128, 32, seed=9, sig_lo=0.08, sig_hi=0.15)
    res = tmp_path / "res"
    res.mkdir()
    fg.write_fvecs(tmp_path / "base.fvecs", x)
    r = subprocess.run([os.path.join(BIN, "build_global"), str(tmp_path / "base.fvecs"), "--res", str(res),
                        "--nlist", "64", "--iters", "5", "--pq_iters", "3", "--sample", "5000", "--no-rebalance"],
                       capture_output=True, text=True, timeout=120, cwd=tmp_path)
    assert r.returncode == 0, r.stderr[-2000:]
    r = subprocess.run([os.path.join(BIN, "tune_parameters"), str(tmp_path / "base.fvecs"), "-n", "300", "-k", "10",
                        "-o", str(tmp_path / "cfg.txt"), "--res", str(res), "--seed", "7", "--samples_out",
                        str(tmp_path / "s.ivecs")], capture_output=True, text=True, timeout=120, cwd=tmp_path)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    cfg = dict(re.findall(r"^([A-Z_0-9]+)=(\S+)$", (tmp_path / "cfg.txt").read_text(), re.M))
    samples = np.fromfile(tmp_path / "s.ivecs", np.int32).reshape(-1, 2)[:, 1]
    assert samples.shape[0] == 300 and samples.min() >= 0 and samples.max() < 20000
    offs, ids, codes, cent = fg.read_ivf_data(res / "ivf_data.bin", 32, 128)
    cb = np.fromfile(res / "global_pq_codebook.bin", np.float32).reshape(32, 256, 4)
    top_m, p1, limit_k, coeff = oracle.tune_parameters(x, offs, ids, codes, cent, cb, samples, 10)
    assert int(cfg["RECOMMENDED_TOP_M"]) == top_m
    assert int(cfg["RECOMMENDED_P1_LISTS"]) == p1
    assert int(cfg["RECOMMENDED_LIMIT_K"]) == limit_k
    assert cfg["THRESHOLD_COEFF"] == f"{coeff:.3f}"
    # the same seed samples the same rows
    r2 = subprocess.run([os.path.join(BIN, "tune_parameters"), str(tmp_path / "base.fvecs"), "-n", "300", "-o",
                         str(tmp_path / "cfg2.txt"), "--res", str(res), "--seed", "7"], capture_output=True, text=True,
                        timeout=120, cwd=tmp_path)
    assert r2.returncode == 0 and (tmp_path / "cfg2.txt").read_text() == (tmp_path / "cfg.txt").read_text()
