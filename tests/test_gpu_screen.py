"""GPU parity of fgpu_search's MFMA screen path: bf16 MFMA distance bounds
pick candidates, which are rescored with the reference's exact LUT arithmetic
(gpu_global.cu:115-158 for the entries, :196-253 for the ascending-m sum).
Bar: ids and fp32 distance bits equal to the oracle's exhaustive scan of the
probed lists, and equal to the same index's LUT kernels (OPT_SCREEN 0), for
every geometry the screen has, k from 1 to 64 (64 round-1 groups above 32),
and every hand-off to the LUT kernel: no threshold (the first usable list
holds fewer than k vectors, or fewer than k of its groups hold a vector), too
many candidates, norms beyond the bounds' range, a misaligned query array.
The screen's counters show which path each case took."""
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


def _gmm_index(dim, m, nlist, n, seed, scale=1.0):
    x = fg.gen_gmm(n, dim, 32, seed=seed, sig_lo=0.08) * np.float32(scale)
    offs, ids, codes, cent, cb = fg.build_ivfpq(torch.from_numpy(x).cuda(), nlist, m, kmeans_iters=4, init_mode=1,
                                                seed=seed, pq_iters=3, sample_size=4000)
    return offs, ids, codes, cent, cb


def _check(idx, q, cent, cb, offs, ids, codes, nprobe, k, prune_ratio=100.0, dq=None, screened=True):
    """Search through the screen (when the index takes it) and the LUT kernels; both against the oracle.
    With screened, the screen's counters of the first search."""
    nq = q.shape[0]
    dq = torch.from_numpy(q).cuda() if dq is None else dq
    ws = torch.empty(max(1, idx.search_workspace_bytes(nq, nprobe)), dtype=torch.uint8, device="cuda")
    sid, sd = idx.search(dq, nprobe, k, prune_ratio=prune_ratio, workspace=ws)
    sid, sd = _host(sid), _host(sd)
    st = idx.search_screen_stats(nq, nprobe, ws) if screened else None
    idx.set_option(fg.Index.OPT_SCREEN, 0)
    lid, ld = idx.search(dq, nprobe, k, prune_ratio=prune_ratio)
    idx.set_option(fg.Index.OPT_SCREEN, 1)
    lid, ld = _host(lid), _host(ld)
    probes, _ = oracle.coarse(q, cent, nprobe, prune_ratio)
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, codes, probes, k)
    bad = np.nonzero(~np.all(sid == oid, axis=1))[0]
    assert bad.size == 0, f"first mismatching queries {bad[:5]}: gpu {sid[bad[0]]} oracle {oid[bad[0]]}"
    assert np.array_equal(_bits(sd), _bits(od))
    assert np.array_equal(lid, oid) and np.array_equal(_bits(ld), _bits(od))
    assert idx.faults() == 0
    return st


@pytest.mark.parametrize("dim,m,k", [(128, 32, 10), (128, 16, 32), (128, 64, 5), (96, 48, 1), (128, 32, 32),
                                     (96, 48, 17), (128, 32, 50), (96, 48, 64), (128, 16, 33)])
def test_screen_geometries_bit_exact(dim, m, k):
    _say(f"screen dim={dim} m={m} k={k}")
    offs, ids, codes, cent, cb = _gmm_index(dim, m, 64, 24000, seed=dim + m + k)
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    assert idx.screen_ready
    q = fg.gen_gmm(333, dim, 32, seed=dim + m + k, set=1, sig_lo=0.08)
    st = _check(idx, q, cent, cb, offs, ids, codes, 12, k)
    # the screen ran: every query whose first list holds k vectors got a
    # threshold from it; queries past 512 candidates (a few, at 16 subspaces
    # and k 32) went to the LUT kernel
    lens = np.diff(offs)
    probes, _ = oracle.coarse(q, cent, 12)
    first = np.array([next((lens[l] for l in row if l < 64 and lens[l] > 0), 0) for row in probes])
    assert st["queries_with_threshold"] == int((first >= k).sum()) >= 333 * 9 // 10
    assert st["candidates"] >= st["queries_with_threshold"] * k
    assert (st["queries_to_lut_kernel"] > int((first < k).sum())) == (st["max_candidates"] > 512)
    # (at k 64, 12 probes of 375-vector lists often pass 512 candidates)
    assert st["queries_to_lut_kernel"] <= 333 // (10 if k <= 32 else 3)
    idx.close()


@pytest.mark.parametrize("nq", [1, 31, 33, 1000])
def test_screen_query_counts_and_pruned_probes(nq):
    """Query counts off the 32-row tile, and coarse pruning (prune_ratio 1.2)
    leaving pruned-probe sentinels in the probe lists."""
    _say(f"screen nq={nq} prune 1.2")
    offs, ids, codes, cent, cb = _gmm_index(128, 32, 128, 30000, seed=nq)
    idx = fg.Index.from_arrays(128, 32, offs, ids, codes, cent, cb)
    q = fg.gen_gmm(nq, 128, 32, seed=nq, set=1, sig_lo=0.08)
    st = _check(idx, q, cent, cb, offs, ids, codes, 24, 10, prune_ratio=1.2)
    probes, _ = oracle.coarse(q, cent, 24, 1.2)
    assert np.any(probes == 0xFFFFFFFF)
    assert st["queries_with_threshold"] == nq
    idx.close()


def test_empty_query_batch():
    """A batch of no queries (arrays that may be null) returns empty results
    from every search entry point."""
    _say("empty batch")
    x = fg.gen_gmm(8000, 128, 32, seed=5, sig_lo=0.08)
    offs, ids, codes, cent, cb = _gmm_index(128, 32, 32, 8000, seed=5)
    idx = fg.Index.from_arrays(128, 32, offs, ids, codes, cent, cb)
    q0 = torch.empty((0, 128), dtype=torch.float32, device="cuda")
    gid, gd = idx.search(q0, 8, 10)
    assert tuple(gid.shape) == (0, 10) and tuple(gd.shape) == (0, 10)
    pid, pd = idx.coarse_search(q0, 8)
    assert tuple(pid.shape) == (0, 8)
    gid, gd = idx.adc_search(q0, pid, 10)
    assert tuple(gid.shape) == (0, 10)
    tid, td, tc, _, _ = idx.two_phase_search(q0, pid, 4, 50, 1.0, 100)
    assert tuple(tid.shape) == (0, 100) and tuple(tc.shape) == (0,)
    gid, gd = idx.search_rerank(q0, torch.from_numpy(x).cuda(), 8, 10, rerank_m=100)
    assert tuple(gid.shape) == (0, 10)
    torch.cuda.synchronize()
    idx.close()


def test_screen_hands_short_first_lists_to_the_lut_kernel():
    """Lists shorter than k: a query whose first non-empty probed list holds
    fewer than k vectors has no threshold and runs the LUT kernel; empty
    lists before it are passed over."""
    _say("screen short first lists")
    rng = np.random.default_rng(7)
    dim, m, nlist, k = 128, 32, 300, 32
    offs, ids, codes, cent, cb = _gmm_index(dim, m, nlist, 9000, seed=7)
    lens = np.diff(offs)
    assert (lens < k).sum() > 20              # many lists shorter than k
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    q = fg.gen_gmm(400, dim, 32, seed=7, set=1, sig_lo=0.08)
    q[:50] = cent[np.argsort(lens)[:50]] + rng.standard_normal((50, dim)).astype(np.float32) * 1e-3
    st = _check(idx, q, cent, cb, offs, ids, codes, 16, k)
    probes, _ = oracle.coarse(q, cent, 16)
    first = np.array([next((lens[l] for l in row if l < nlist and lens[l] > 0), 0) for row in probes])
    assert st["queries_with_threshold"] == int((first >= k).sum())
    assert st["queries_to_lut_kernel"] >= int(((first > 0) & (first < k)).sum()) > 0
    idx.close()


def test_screen_single_probe_short_and_empty_lists():
    """nprobe 1: a query whose only list holds fewer than k vectors takes them
    all as its candidates, one whose list is empty gets padding; neither runs
    the LUT kernel.  Bit-exact with the oracle and the LUT kernels."""
    _say("screen single probe, short and empty lists")
    rng = np.random.default_rng(13)
    dim, m, nlist, k = 128, 32, 300, 32
    offs, ids, codes, cent, cb = _gmm_index(dim, m, nlist, 9000, seed=13)
    lens = np.diff(offs)
    empty = np.argsort(np.where(lens > 0, lens, 1 << 30))[:5]  # the five shortest lists, emptied
    keep = np.ones(len(ids), bool)
    for e in empty:
        keep[offs[e]:offs[e + 1]] = False
    lens2 = lens.copy()
    lens2[empty] = 0
    offs2 = np.concatenate([[0], np.cumsum(lens2)]).astype(offs.dtype)
    ids2, codes2 = np.ascontiguousarray(ids[keep]), np.ascontiguousarray(codes[keep])
    idx = fg.Index.from_arrays(dim, m, offs2, ids2, codes2, cent, cb)
    assert idx.screen_ready
    short = np.nonzero((lens2 > 0) & (lens2 < k))[0]
    assert short.size >= 10
    pick = np.concatenate([empty, short[:20]])
    q = cent[np.repeat(pick, 3)] + rng.standard_normal((3 * pick.size, dim)).astype(np.float32) * 1e-3
    q = np.concatenate([q, fg.gen_gmm(100, dim, 32, seed=13, set=1, sig_lo=0.08)]).astype(np.float32)
    st = _check(idx, q, cent, cb, offs2, ids2, codes2, 1, k)
    probes, _ = oracle.coarse(q, cent, 1)
    n1 = lens2[probes[:, 0]]
    assert (n1 == 0).sum() >= 10 and ((n1 > 0) & (n1 < k)).sum() >= 30
    assert st["queries_with_threshold"] == int((n1 >= k).sum())
    assert st["queries_to_lut_kernel"] == 0
    idx.close()


def test_screen_hands_candidate_overflow_to_the_lut_kernel():
    """A list of several hundred vectors sharing one code: every one ties with the
    nearest, so the query's candidates pass 512 and it runs the LUT kernel;
    the (distance, id) tie rule still picks the smallest ids."""
    _say("screen candidate overflow")
    rng = np.random.default_rng(11)
    dim, m, nlist, k = 128, 32, 16, 32
    offs, ids, codes, cent, cb = _gmm_index(dim, m, nlist, 12000, seed=11)
    big = int(np.argmax(np.diff(offs)))
    codes = codes.copy()
    s, e = offs[big], offs[big + 1]
    assert e - s > 600
    codes[s:e] = codes[s]
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    q = np.repeat(cent[big:big + 1], 40, axis=0) + rng.standard_normal((40, dim)).astype(np.float32) * 1e-2
    q = np.concatenate([q, fg.gen_gmm(60, dim, 32, seed=11, set=1, sig_lo=0.08)]).astype(np.float32)
    st = _check(idx, q, cent, cb, offs, ids, codes, 4, k)
    assert st["queries_to_lut_kernel"] >= 40
    assert st["max_candidates"] > 512
    idx.close()


@pytest.mark.parametrize("nprobe", [32, 27])
def test_screen_every_probe_passes_round_2(nprobe):
    """One Gaussian blob split into 32 lists: every list's bound is below each
    query's threshold, so round 2 takes (almost) every probe, and the pair
    kernel builds the A fragments of many probes a query, several batches of
    centroid rows (the last one partial at 27 probes)."""
    _say(f"screen all probes pass, nprobe={nprobe}")
    dim, m, nlist, k = 128, 32, 32, 10
    x = fg.gen_gmm(16000, dim, 1, seed=5, sig_lo=0.08)
    offs, ids, codes, cent, cb = fg.build_ivfpq(torch.from_numpy(x).cuda(), nlist, m, kmeans_iters=4, init_mode=1,
                                                seed=5, pq_iters=3, sample_size=4000)
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    q = fg.gen_gmm(200, dim, 1, seed=5, set=1, sig_lo=0.08)
    st = _check(idx, q, cent, cb, offs, ids, codes, nprobe, k)
    assert st["queries_with_threshold"] == 200
    assert st["pairs_round2"] >= 200 * nprobe * 9 // 10
    idx.close()


@pytest.mark.parametrize("scale", [300.0, 1e-3])
def test_screen_scaled_data(scale):
    """Large (x 300, norms^2 near 1e7) and small (x 1e-3) data: the bounds'
    relative and absolute slack both hold; the screen still runs."""
    _say(f"screen scale {scale}")
    offs, ids, codes, cent, cb = _gmm_index(128, 32, 64, 20000, seed=3, scale=scale)
    idx = fg.Index.from_arrays(128, 32, offs, ids, codes, cent, cb)
    assert idx.screen_ready
    q = fg.gen_gmm(300, 128, 32, seed=3, set=1, sig_lo=0.08) * np.float32(scale)
    st = _check(idx, q, cent, cb, offs, ids, codes, 12, 10)
    assert st["queries_with_threshold"] == 300
    idx.close()


def test_screen_off_beyond_its_norm_range():
    """Decoded vector norms above 2^40: the index carries no screen and
    search runs the LUT kernels.  Query residual norms above 2^40 on an index
    with the screen: those queries get no threshold and run the LUT kernel.
    Results unchanged either way."""
    _say("screen norm range")
    offs, ids, codes, cent, cb = _gmm_index(128, 32, 32, 8000, seed=9)
    big = np.float32(2.0 ** 42)
    idx = fg.Index.from_arrays(128, 32, offs, ids, codes, cent * big, cb * big)
    assert not idx.screen_ready
    q = fg.gen_gmm(100, 128, 32, seed=9, set=1, sig_lo=0.08)
    _check(idx, q * big, cent * big, cb * big, offs, ids, codes, 8, 10, screened=False)
    idx.close()
    idx = fg.Index.from_arrays(128, 32, offs, ids, codes, cent, cb)
    assert idx.screen_ready
    q[:7] *= np.float32(2.0 ** 41)
    st = _check(idx, q, cent, cb, offs, ids, codes, 8, 10)
    assert st["queries_with_threshold"] == 93 and st["queries_to_lut_kernel"] == 7
    idx.close()


def test_screen_row_scales_for_far_queries():
    """Queries far from the data: each pair row of the fp16 screen runs at its
    own power-of-two scale (its residual norm squared over 2^14), so a query
    tens of data radii away still takes the screen; one whose row would need
    more than 2^14 takes the LUT kernel.  Bit-exact either way."""
    _say("screen row scales, far queries")
    rng = np.random.default_rng(21)
    offs, ids, codes, cent, cb = _gmm_index(128, 32, 64, 20000, seed=21)
    idx = fg.Index.from_arrays(128, 32, offs, ids, codes, cent, cb)
    assert idx.screen_ready
    q = fg.gen_gmm(200, 128, 32, seed=21, set=1, sig_lo=0.08)
    spread = float(np.linalg.norm(cent - cent.mean(axis=0), axis=1).max())
    d = rng.standard_normal(128).astype(np.float32)
    d /= np.linalg.norm(d)
    q[:60] += d * np.float32(30.0 * spread)      # far: larger row scales, still screened
    q[60:70] += d * np.float32(3.0e5 * spread)   # beyond the row scales: the LUT kernel
    q = q.astype(np.float32)
    st = _check(idx, q, cent, cb, offs, ids, codes, 8, 10)
    assert st["queries_with_threshold"] == 190
    assert st["queries_to_lut_kernel"] >= 10
    idx.close()


def test_screen_misaligned_queries_take_the_lut_kernel():
    """A query array 4 bytes off 16-byte alignment: the screen's vector loads
    need 16, so search takes the LUT kernels, results unchanged."""
    _say("screen misaligned queries")
    offs, ids, codes, cent, cb = _gmm_index(128, 32, 32, 8000, seed=13)
    idx = fg.Index.from_arrays(128, 32, offs, ids, codes, cent, cb)
    q = fg.gen_gmm(70, 128, 32, seed=13, set=1, sig_lo=0.08)
    buf = torch.empty(q.size + 1, dtype=torch.float32, device="cuda")
    dq = buf[1:].view(70, 128)
    dq.copy_(torch.from_numpy(q))
    assert dq.data_ptr() % 16 == 4
    _check(idx, q, cent, cb, offs, ids, codes, 8, 10, dq=dq, screened=False)
    idx.close()


@pytest.mark.parametrize("k", [33, 48, 64])
def test_screen_k_above_32_uses_64_groups(k):
    """k in (32, 64]: round 1 keeps 64 group minima a row; every query still gets a threshold from its first
    list (lists of about 250 vectors, so all 64 groups hold one)."""
    _say(f"screen k {k}")
    offs, ids, codes, cent, cb = _gmm_index(128, 32, 32, 8000, seed=17)
    idx = fg.Index.from_arrays(128, 32, offs, ids, codes, cent, cb)
    q = fg.gen_gmm(90, 128, 32, seed=17, set=1, sig_lo=0.08)
    st = _check(idx, q, cent, cb, offs, ids, codes, 8, k)
    assert st["queries_with_threshold"] == 90 and st["pairs_round1"] == 90
    idx.close()
