"""GPU parity: the HIP path (through the C ABI) against the CPU oracle on the
same seeded inputs.  Bar: bit-exact ids, codes, assignments and -- because
every distance is computed in the reference's exact operation order --
bit-exact fp32 distances too (the north-star tolerance is 1e-4 relative).
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
from tests.golden.make_golden import inputs as golden_inputs  # noqa: E402


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _random_index(rng, n, dim, m, nlist, empty=(), big=None):
    """A valid index with arbitrary codes: list sizes skewed, some empty, one very long."""
    p = rng.random(nlist) + 0.05
    for e in empty:
        p[e] = 0.0
    if big is not None:
        p[big] *= 40.0
    assign = rng.choice(nlist, size=n, p=p / p.sum()).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    codes[100] = codes[101]            # exact ADC ties ...
    assign[101] = assign[100]          # ... inside one list
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = rng.standard_normal((nlist, dim)).astype(np.float32) * 0.7
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    return offs, ids, lc, cent, cb


# --------------------------------------------------------------------------- exact nearest centroids
@pytest.mark.parametrize("dim,nc,p", [(128, 1024, 32), (96, 300, 1), (128, 4096, 64), (64, 50, 10), (128, 77, 1),
                                      (36, 200, 8), (128, 4096, 1), (96, 2500, 1), (36, 1111, 1)])
def test_l2_topk_bit_exact(dim, nc, p):
    _say(f"l2_topk dim={dim} nc={nc} p={p}")
    rng = np.random.default_rng(dim + nc + p)
    x = rng.standard_normal((257, dim)).astype(np.float32)
    c = rng.standard_normal((nc, dim)).astype(np.float32)
    c[5] = c[2]                      # duplicate centroid -> exact ties
    x[3] = c[2]                      # distance 0 to two centroids
    x[4] = c[2] + np.float32(1e-3)   # near-tie region for the GEMM estimate
    ids, d = fg.l2_topk(torch.from_numpy(x).cuda(), torch.from_numpy(c).cuda(), p)
    ids, d = _host(ids), _host(d)
    oid, od = oracle.coarse(x, c, p, prune_ratio=np.inf)  # best*inf never prunes (0*inf is NaN)
    assert np.array_equal(ids.view(np.uint32), oid)
    assert np.array_equal(_bits(d), _bits(od))
    if p == 1:
        assert np.array_equal(ids[:, 0], oracle.kmeans_assign(x, c))


@pytest.mark.parametrize("case", ["large", "tiny", "sphere", "offset"])
@pytest.mark.parametrize("dim,p,nc", [(128, 32, 1024), (128, 1, 1024), (36, 8, 1024), (128, 1, 3000)])
def test_l2_topk_estimate_extremes(case, dim, p, nc):
    """The select reads fp16 lower bounds of the shifted estimates, each row
    scaled by a power of two into the fp16 range: large values (x 300), values
    in the fp16 subnormal range, many near-equal distances (a query at the
    centre of a sphere of centroids) and a large common offset of both sets
    (estimates far from zero against small differences) all stay exact."""
    _say(f"l2_topk extremes case={case} dim={dim} p={p} nc={nc}")
    rng = np.random.default_rng(["large", "tiny", "sphere", "offset"].index(case) * 1000 + dim * 10 + p + nc)
    n = 129
    x = rng.standard_normal((n, dim)).astype(np.float32)
    c = rng.standard_normal((nc, dim)).astype(np.float32)
    if case == "large":
        x *= np.float32(300.0)
        c *= np.float32(300.0)
    elif case == "tiny":
        x *= np.float32(2e-3)
        c *= np.float32(2e-3)
    elif case == "sphere":
        u = c / np.linalg.norm(c, axis=1, keepdims=True)
        c = (x[0] + np.float32(0.5) * u).astype(np.float32)
        x[1:] = x[0] + np.float32(1e-4) * rng.standard_normal((n - 1, dim)).astype(np.float32)
    else:
        off = rng.standard_normal(dim).astype(np.float32) * np.float32(30.0)
        x += off
        c += off
    ids, d = fg.l2_topk(torch.from_numpy(x).cuda(), torch.from_numpy(c).cuda(), p)
    ids, d = _host(ids), _host(d)
    oid, od = oracle.coarse(x, c, p, prune_ratio=np.inf)
    assert np.array_equal(ids.view(np.uint32), oid)
    assert np.array_equal(_bits(d), _bits(od))


# --------------------------------------------------------------------------- coarse quantizer (A2, A3)
@pytest.mark.parametrize("case", ["unit", "x300", "sift_like"])
def test_coarse_margin_stays_tight_at_large_norms(case):
    """Large norms do not turn the coarse step into a brute-force re-score:
    the fp16 estimates of each row are scaled into range, so the margin still
    admits few centroids per query (unit-scale mixture data, the same x 300,
    and SIFT-like data with every coordinate in [0, 255] and squared norms
    near 2e6); results bit-exact."""
    _say(f"coarse margin case={case}")
    rng = np.random.default_rng(["unit", "x300", "sift_like"].index(case) + 77)
    if case == "sift_like":
        x = fg.gen_gmm(20000, 128, 64, seed=8, lo=0.0, hi=200.0, sig_lo=12.0)
        q = fg.gen_gmm(500, 128, 64, seed=8, set=1, lo=0.0, hi=200.0, sig_lo=12.0)
        x, q = np.clip(x, 0, 255).round(), np.clip(q, 0, 255).round()
    else:
        sc = np.float32(300.0 if case == "x300" else 1.0)
        x = fg.gen_gmm(20000, 128, 64, seed=8, sig_lo=0.1) * sc
        q = fg.gen_gmm(500, 128, 64, seed=8, set=1, sig_lo=0.1) * sc
    x, q = x.astype(np.float32), q.astype(np.float32)
    cent = x[rng.choice(x.shape[0], 1024, replace=False)].copy()
    offs, ids, lc, _, cb = _random_index(rng, 4000, 128, 32, 1024)
    idx = fg.Index.from_arrays(128, 32, offs, ids, lc, cent, cb)
    pid, pd, st = idx.coarse_search_stats(torch.from_numpy(q).cuda(), 32)
    pid, pd = _host(pid).view(np.uint32), _host(pd)
    oid, od = oracle.coarse(q, cent, 32)
    assert np.array_equal(pid, oid) and np.array_equal(_bits(pd), _bits(od))
    per_q = st["rescored"] / q.shape[0]
    _say(f"  {per_q:.1f} centroids re-scored a query, {st['full_rows']} queries re-scored all 1024")
    assert st["full_rows"] == 0 and per_q < 160, st
    idx.close()


@pytest.mark.parametrize("prune_ratio", [100.0, 1.3])
def test_coarse_search_bit_exact(prune_ratio):
    _say(f"coarse prune_ratio={prune_ratio}")
    rng = np.random.default_rng(3)
    offs, ids, lc, cent, cb = _random_index(rng, 4000, 128, 32, 256)
    cent[9] = cent[4]
    q = rng.standard_normal((300, 128)).astype(np.float32) * 0.7
    q[0] = cent[4]
    idx = fg.Index.from_arrays(128, 32, offs, ids, lc, cent, cb)
    pid, pd = idx.coarse_search(torch.from_numpy(q).cuda(), 32, prune_ratio)
    pid, pd = _host(pid).view(np.uint32), _host(pd)
    oid, od = oracle.coarse(q, cent, 32, prune_ratio)
    assert np.array_equal(pid, oid)
    assert np.array_equal(_bits(pd), _bits(od))
    idx.close()


@pytest.mark.parametrize("p,prune_ratio", [(100, 1.3), (256, float("inf")), (65, 100.0)])
def test_coarse_search_many_probes(p, prune_ratio):
    """Top-p above one 64-key list (up to four lists merged in cascade),
    with duplicate centroids for ties and the prune rule past rank 64."""
    _say(f"coarse p={p} prune_ratio={prune_ratio}")
    rng = np.random.default_rng(p)
    offs, ids, lc, cent, cb = _random_index(rng, 6000, 128, 32, 700)
    cent[9] = cent[4]
    cent[300] = cent[200]
    q = rng.standard_normal((200, 128)).astype(np.float32) * 0.7
    q[0] = cent[4]
    idx = fg.Index.from_arrays(128, 32, offs, ids, lc, cent, cb)
    pid, pd = idx.coarse_search(torch.from_numpy(q).cuda(), p, prune_ratio)
    pid, pd = _host(pid).view(np.uint32), _host(pd)
    oid, od = oracle.coarse(q, cent, p, prune_ratio)
    assert np.array_equal(pid, oid)
    assert np.array_equal(_bits(pd), _bits(od))
    idx.close()


# --------------------------------------------------------------------------- LUT + ADC + top-k (A4-A6, A10)
@pytest.mark.parametrize("dim,m,p", [(128, 32, 65), (128, 16, 100), (96, 32, 256), (96, 16, 77)])
def test_search_more_than_64_probes(dim, m, p):
    """nprobe above the flow kernel's 64-list tables: fgpu_search (coarse +
    scan) and fgpu_adc_search run the barrier-per-list kernel, which scans
    every probed list, pruned probes included as skips."""
    _say(f"search dim={dim} m={m} nprobe={p}")
    rng = np.random.default_rng(dim + m + p)
    offs, ids, lc, cent, cb = _random_index(rng, 9000, dim, m, 300)
    q = rng.standard_normal((120, dim)).astype(np.float32) * 0.7
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    dq = torch.from_numpy(q).cuda()
    gid, gd = idx.search(dq, p, 10, prune_ratio=1.5)
    probes, _ = oracle.coarse(q, cent, p, 1.5)
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, 10)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    gid, gd = idx.adc_search(dq, torch.from_numpy(probes.view(np.int32)).cuda(), 10)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    idx.check()
    idx.close()


@pytest.mark.parametrize("dim,m,k", [(128, 32, 10), (128, 16, 10), (96, 48, 20), (96, 32, 64), (128, 64, 1),
                                     (96, 16, 7)])
def test_adc_search_bit_exact(dim, m, k):
    _say(f"adc dim={dim} m={m} k={k}")
    rng = np.random.default_rng(dim * m + k)
    nlist = 40
    offs, ids, lc, cent, cb = _random_index(rng, 30000, dim, m, nlist, empty=(3, 17), big=8)
    q = rng.standard_normal((150, dim)).astype(np.float32) * 0.7
    probes, pdist = oracle.coarse(q, cent, 12)
    probes[5, 2] = 0xFFFFFFFF             # pruned probe mid-list
    probes[6, :] = 0xFFFFFFFF             # every probe pruned -> padding
    probes[7, 0] = 3                      # an empty list first
    probes[8, :] = probes[8, 0]           # the same list probed twice is scanned twice
    pdist[8, :] = pdist[8, 0]
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    assert idx.max_list_len > 1024        # longer than the reference's 1024-item cut
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, k)
    # list bounds from the centroids, then from the coarse distances
    for pd in (None, torch.from_numpy(pdist).cuda()):
        gid, gd = idx.adc_search(torch.from_numpy(q).cuda(), torch.from_numpy(probes.view(np.int32)).cuda(), k,
                                 probe_dists=pd)
        gid, gd = _host(gid), _host(gd)
        bad = np.nonzero(~np.all(gid == oid, axis=1))[0]
        assert bad.size == 0, f"first mismatching queries {bad[:5]}: gpu {gid[bad[0]]} oracle {oid[bad[0]]}"
        assert np.array_equal(_bits(gd), _bits(od))
        assert np.all(gid[6] == -1)
    assert idx.faults() == 0
    idx.close()


@pytest.mark.parametrize("dim,m,k", [(128, 32, 10), (96, 16, 33)])
def test_adc_search_many_queries_per_workgroup(dim, m, k):
    """More queries than resident workgroups: each workgroup runs a dozen
    queries back to back through its two per-query state slots."""
    _say(f"adc many queries dim={dim} m={m} k={k}")
    rng = np.random.default_rng(dim + m + k + 5)
    nlist = 64
    offs, ids, lc, cent, cb = _random_index(rng, 40000, dim, m, nlist, empty=(5,), big=9)
    nq = 3000
    q = rng.standard_normal((nq, dim)).astype(np.float32) * 0.7
    probes, pdist = oracle.coarse(q, cent, 16)
    probes[300:303, :] = 0xFFFFFFFF       # consecutive queries with nothing to scan
    probes[700, 1:] = 0xFFFFFFFF          # one list only
    probes[1500, :] = probes[1500, 0]     # one list, probed 16 times
    pdist[1500, :] = pdist[1500, 0]
    probes[2999, 0] = 5                   # an empty list first, on the last query
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, k)
    for pd in (None, torch.from_numpy(pdist).cuda()):
        gid, gd = idx.adc_search(torch.from_numpy(q).cuda(), torch.from_numpy(probes.view(np.int32)).cuda(), k,
                                 probe_dists=pd)
        gid, gd = _host(gid), _host(gd)
        bad = np.nonzero(~np.all(gid == oid, axis=1))[0]
        assert bad.size == 0, f"first mismatching queries {bad[:5]}: gpu {gid[bad[0]]} oracle {oid[bad[0]]}"
        assert np.array_equal(_bits(gd), _bits(od))
        assert np.all(gid[300:303] == -1)
    assert idx.faults() == 0
    idx.close()


def test_search_fused_equals_stages():
    _say("fused search")
    rng = np.random.default_rng(21)
    offs, ids, lc, cent, cb = _random_index(rng, 20000, 128, 32, 128)
    q = torch.from_numpy(rng.standard_normal((500, 128)).astype(np.float32) * 0.7).cuda()
    idx = fg.Index.from_arrays(128, 32, offs, ids, lc, cent, cb)
    fid, fd = idx.search(q, 16, 10)
    pid, pdist = idx.coarse_search(q, 16)
    sid, sd = idx.adc_search(q, pid, 10)
    assert torch.equal(fid, sid) and torch.equal(fd, sd)
    sid, sd = idx.adc_search(q, pid, 10, probe_dists=pdist)
    assert torch.equal(fid, sid) and torch.equal(fd, sd)
    qn = q.cpu().numpy()
    oprobe, _ = oracle.coarse(qn, cent, 16)
    oid, od = oracle.search_plain(qn, cent, cb, offs, ids, lc, oprobe, 10)
    assert np.array_equal(_host(fid), oid) and np.array_equal(_bits(_host(fd)), _bits(od))
    cnt, off = fg.probe_counts(idx, pid)
    ocnt = oracle.probe_counts(oprobe, offs)
    assert np.array_equal(_host(cnt), ocnt)
    assert np.array_equal(_host(off), np.concatenate([[0], np.cumsum(ocnt)]).astype(np.int32))
    assert idx.faults() == 0
    idx.close()


# --------------------------------------------------------------------------- k-means (A13, A14)
def test_kmeans_update_bit_exact():
    _say("kmeans_update")
    rng = np.random.default_rng(31)
    x = rng.standard_normal((20000, 128)).astype(np.float32)
    k = 50
    a = rng.integers(0, k - 1, 20000).astype(np.int32)
    old = rng.standard_normal((k, 128)).astype(np.float32)
    shift = fg.fixed_shift(float(np.abs(x).max()), x.shape[0])
    for rule in (0, 1):
        c = torch.from_numpy(old.copy()).cuda()
        cnt = fg.kmeans_update(torch.from_numpy(x).cuda(), torch.from_numpy(a).cuda(), c, shift, rule)
        want, wcnt = oracle.kmeans_update(x, a, old, shift, rule)
        assert np.array_equal(_host(cnt), wcnt)
        assert np.array_equal(_bits(_host(c)), _bits(want))


@pytest.mark.parametrize("init_mode", [0, 1])
def test_kmeans_fit_bit_exact(init_mode):
    _say(f"kmeans_fit init={init_mode}")
    x = oracle.gen_gmm(6000, 128, 24, seed=5, sig_lo=0.1)
    cent, assign = fg.kmeans_fit(torch.from_numpy(x).cuda(), 48, 6, init_mode=init_mode, seed=42)
    oc, oa = oracle.kmeans_fit(x, 48, 6, init_mode=init_mode, seed=42)
    assert np.array_equal(_bits(_host(cent)), _bits(oc))
    assert np.array_equal(_host(assign), oa)


@pytest.mark.parametrize("n,dim,comp,k", [(40000, 128, 64, 300), (20000, 96, 40, 200), (8000, 40, 16, 120)])
def test_kmeans_pp_seeding_bit_exact(n, dim, comp, k):
    """k-means++ seeding (iters = 0) on tight clusters with duplicate rows, so
    the update's exact triangle-inequality skip clears most rows after the
    first picks: the centres equal the oracle's unpruned definition bit for
    bit (dims 128 and 96 take the vectorised kernel, 40 the generic one)."""
    _say(f"kmeans++ seeding n={n} dim={dim} k={k}")
    x = oracle.gen_gmm(n, dim, comp, seed=17, sig_lo=0.05)
    x[-200:] = x[:200]  # duplicates: rows at distance 0 from a picked centre
    cent, _ = fg.kmeans_fit(torch.from_numpy(x).cuda(), k, 0, init_mode=1, seed=7, want_assign=False)
    want, rows = oracle.kmeans_init_pp(x, k, 7)
    assert len(set(rows.tolist())) == k
    assert np.array_equal(_bits(_host(cent)), _bits(want))


# --------------------------------------------------------------------------- PQ (A15, A16)
def test_pq_train_matches_reference_fixture():
    _say("pq_train golden")
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_pq.npz"))
    _, x, cent, assign = golden_inputs()
    cb = fg.pq_train(torch.from_numpy(x).cuda(), torch.from_numpy(assign).cuda(), torch.from_numpy(cent).cuda(),
                     32, sample_size=500, iters=5)
    assert np.array_equal(_bits(_host(cb)), _bits(g["codebook"]))


@pytest.mark.parametrize("dim,m", [(128, 32), (128, 16), (96, 48)])
def test_pq_train_and_encode_bit_exact(dim, m):
    _say(f"pq dim={dim} m={m}")
    rng = np.random.default_rng(dim + m)
    nlist = 20
    cent = rng.standard_normal((nlist, dim)).astype(np.float32)
    a = rng.integers(0, nlist, 5000).astype(np.int32)
    x = (cent[a] + 0.3 * rng.standard_normal((5000, dim))).astype(np.float32)
    dx, da, dc = torch.from_numpy(x).cuda(), torch.from_numpy(a).cuda(), torch.from_numpy(cent).cuda()
    cb = fg.pq_train(dx, da, dc, m, sample_size=3000, iters=4)
    ocb = oracle.pq_train(x, a, cent, m, sample_size=3000, iters=4)
    assert np.array_equal(_bits(_host(cb)), _bits(ocb))
    codes = fg.pq_encode(dx, da, dc, cb)
    assert np.array_equal(_host(codes), oracle.pq_encode(x, a, cent, ocb, fma_mode=1))


def test_build_ivfpq_bit_exact():
    _say("build_ivfpq")
    x = oracle.gen_gmm(8000, 128, 16, seed=9, sig_lo=0.1)
    got = fg.build_ivfpq(torch.from_numpy(x).cuda(), 32, 32, kmeans_iters=4, init_mode=1, seed=7, pq_iters=3,
                         sample_size=3000)
    want = oracle.build_ivfpq(x, 32, 32, kmeans_iters=4, init_mode=1, seed=7, pq_iters=3, sample_size=3000)
    for g, w, name in zip(got, want, ["offsets", "ids", "codes", "centroids", "codebook"]):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8)), name


def test_config1_end_to_end_bit_exact():
    """BASELINE config 1 at full size: 100k x 128 (64-component mixture, sigma 0.1), 256 lists, PQ M=16,
    1000 queries, nprobe 16, k 10 -- index build and search, GPU against the oracle."""
    _say("config 1 end to end")
    x = oracle.gen_gmm(100000, 128, 64, seed=11, sig_lo=0.1)
    q = oracle.gen_gmm(1000, 128, 64, seed=11, set=1, sig_lo=0.1)
    got = fg.build_ivfpq(torch.from_numpy(x).cuda(), 256, 16, kmeans_iters=20, init_mode=1, seed=42, pq_iters=8,
                         sample_size=50000)
    want = oracle.build_ivfpq(x, 256, 16, kmeans_iters=20, init_mode=1, seed=42, pq_iters=8, sample_size=50000)
    for g, w, name in zip(got, want, ["offsets", "ids", "codes", "centroids", "codebook"]):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8)), name
    offs, ids, codes, cent, cb = want
    idx = fg.Index.from_arrays(128, 16, offs, ids, codes, cent, cb)
    gid, gd = idx.search(torch.from_numpy(q).cuda(), 16, 10)
    probes, _ = oracle.coarse(q, cent, 16)
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, codes, probes, 10)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    idx.close()


def test_search_on_a_side_stream():
    """stream= runs the whole call (conversions, workspace, outputs, kernels) on
    that stream; results equal the default stream's."""
    _say("search on a side stream")
    rng = np.random.default_rng(23)
    offs, ids, lc, cent, cb = _random_index(rng, 20000, 128, 32, 128)
    q = rng.standard_normal((700, 128)).astype(np.float32) * 0.7
    idx = fg.Index.from_arrays(128, 32, offs, ids, lc, cent, cb)
    ref_id, ref_d = idx.search(torch.from_numpy(q).cuda(), 16, 10)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    for _ in range(3):  # freed internal buffers are reused on the same stream only
        gid, gd = idx.search(q, 16, 10, stream=s)
        pid, pdist = idx.coarse_search(q, 16, stream=s)
        aid, ad = idx.adc_search(q, pid, 10, probe_dists=pdist, stream=s)
    s.synchronize()
    assert torch.equal(gid, ref_id) and torch.equal(gd, ref_d)
    assert torch.equal(aid, ref_id) and torch.equal(ad, ref_d)
    assert idx.faults(stream=s) == 0
    idx.close()


def test_wrapped_device_arrays_search_like_an_owned_index():
    """fgpu_index_wrap over device arrays the caller holds (the reference's
    IVFIndexGPU) gives the same search as an index that owns copies; the
    in-place prune equals the oracle's prune rule."""
    _say("index wrap + prune_probes")
    rng = np.random.default_rng(31)
    offs, ids, lc, cent, cb = _random_index(rng, 20000, 128, 32, 96)
    q = torch.from_numpy(rng.standard_normal((400, 128)).astype(np.float32) * 0.7).cuda()
    own = fg.Index.from_arrays(128, 32, offs, ids, lc, cent, cb)
    dev = [torch.from_numpy(a).cuda() for a in (offs, ids, lc, cent, cb)]
    wrapped = fg.Index.wrap(128, 32, *dev)
    assert (wrapped.nlist, wrapped.total, wrapped.max_list_len) == (own.nlist, own.total, own.max_list_len)
    a = own.search(q, 16, 10)
    b = wrapped.search(q, 16, 10)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    pid, pd = own.coarse_search(q, 16, prune_ratio=np.inf)
    fg.prune_probes(pid, pd, 1.2)
    oid, _ = oracle.coarse(q.cpu().numpy(), cent, 16, prune_ratio=1.2)
    assert np.array_equal(_host(pid).view(np.uint32), oid)
    assert wrapped.faults() == 0
    wrapped.close()
    own.close()
