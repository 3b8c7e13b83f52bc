"""Seeded random shapes against the oracle, bit for bit: the coarse step,
the plain search (flow kernel) and the two-phase search over random
geometries, list-size skews, empty lists, probe counts (up to 256), k,
p1_lists, limit_k (both phase-1 paths), rerank_m and prune ratios.  Each
case prints its parameters before it runs."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no HIP device", allow_module_level=True)

import fusiongpu_amd as fg  # noqa: E402
import oracle  # noqa: E402

GEOMS = [(128, 32), (128, 16), (128, 64), (96, 48), (96, 32), (96, 16)]


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _case(seed):
    rng = np.random.default_rng(seed)
    dim, m = GEOMS[rng.integers(len(GEOMS))]
    nlist = int(rng.integers(20, 320))
    n = int(rng.integers(5000, 30000))
    p = rng.random(nlist) ** 3 + 0.01  # skewed list sizes
    p[rng.integers(0, nlist, 3)] = 0.0  # a few empty lists
    assign = rng.choice(nlist, size=n, p=p / p.sum()).astype(np.int32)
    x = (rng.standard_normal((n, dim)) * 0.6).astype(np.float32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = (rng.standard_normal((nlist, dim)) * 0.7).astype(np.float32)
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    nq = int(rng.integers(50, 400))
    q = (rng.standard_normal((nq, dim)) * 0.7).astype(np.float32)
    return rng, dim, m, nlist, offs, ids, lc, cent, cb, q, x


@pytest.mark.parametrize("seed", range(100, 112))
def test_random_coarse_and_plain_search(seed):
    rng, dim, m, nlist, offs, ids, lc, cent, cb, q, _ = _case(seed)
    nprobe = int(rng.integers(1, min(nlist, 64) + 1))
    k = int(rng.integers(1, 65))
    prune = float(rng.choice([100.0, 1.2, 1.05, np.inf]))
    _say(f"seed {seed}: plain dim={dim} m={m} nlist={nlist} nq={q.shape[0]} nprobe={nprobe} k={k} prune={prune}")
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    dq = torch.from_numpy(q).cuda()
    pid, pd = idx.coarse_search(dq, nprobe, prune)
    oid, od = oracle.coarse(q, cent, nprobe, prune)
    assert np.array_equal(pid.cpu().numpy().view(np.uint32), oid)
    assert np.array_equal(_bits(pd.cpu().numpy()), _bits(od))
    gid, gd = idx.search(dq, nprobe, k, prune)
    wid, wd = oracle.search_plain(q, cent, cb, offs, ids, lc, oid, k)
    assert np.array_equal(gid.cpu().numpy(), wid)
    assert np.array_equal(_bits(gd.cpu().numpy()), _bits(wd))
    assert idx.faults() == 0
    idx.close()


@pytest.mark.parametrize("seed", range(200, 212))
def test_random_two_phase(seed):
    rng, dim, m, nlist, offs, ids, lc, cent, cb, q, _ = _case(seed)
    nprobe = int(rng.integers(1, min(nlist, 256) + 1))
    p1 = int(rng.integers(0, nprobe + 1))
    limit_k = int(rng.choice([int(rng.integers(1, 65)), int(rng.integers(65, 300))]))
    rerank_m = int(rng.integers(1, 3000))
    coeff = float(rng.choice([0.0, 0.8, 1.0, 1.5, 4.0]))
    _say(f"seed {seed}: two-phase dim={dim} m={m} nlist={nlist} nq={q.shape[0]} nprobe={nprobe} p1={p1} "
         f"limit_k={limit_k} coeff={coeff} rerank_m={rerank_m}")
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    probes, _ = oracle.coarse(q, cent, nprobe)
    gid, gd, gcnt, gcut, gthr = idx.two_phase_search(torch.from_numpy(q).cuda(),
                                                     torch.from_numpy(probes.view(np.int32)).cuda(), p1, limit_k,
                                                     coeff, rerank_m, want_cutoffs=p1 > 0)
    oid, od, ocnt, ocut, othr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, coeff,
                                                        rerank_m)
    assert np.array_equal(gcnt.cpu().numpy(), ocnt)
    assert np.array_equal(gid.cpu().numpy(), oid)
    assert np.array_equal(_bits(gd.cpu().numpy()), _bits(od))
    assert np.array_equal(_bits(gthr.cpu().numpy()), _bits(othr))
    if p1 > 0:
        assert np.array_equal(_bits(gcut.cpu().numpy()), _bits(ocut))
    idx.close()
