"""GPU parity for the two-phase pruned scan (A6-A10) and the exact rerank
(A11): the HIP path through the C ABI against the CPU oracle on the same
seeded inputs.  Bar: bit-exact ids, counts, cutoffs, thresholds, visit counts
and fp32 distances.
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


def _index(rng, n, dim, m, nlist, empty=(), big=None):
    p = rng.random(nlist) + 0.05
    for e in empty:
        p[e] = 0.0
    if big is not None:
        p[big] *= 40.0
    assign = rng.choice(nlist, size=n, p=p / p.sum()).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    codes[100] = codes[101]
    assign[101] = assign[100]
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = rng.standard_normal((nlist, dim)).astype(np.float32) * 0.7
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    return offs, ids, lc, cent, cb


# (dim, m, p1_lists, limit_k, coeff, rerank_m)
CASES = [
    (128, 32, 3, 5, 1.0, 60),      # reference-shaped, small
    (96, 48, 12, 50, 1.0, 1000),   # config-3 shape
    (128, 16, 0, 10, 1.0, 50),     # no phase 1: thr = FLT_MAX, every vector passes, pool selects repeatedly
    (96, 32, 16, 64, 1.5, 300),    # every probe in phase 1
    (128, 64, 4, 1, 0.0, 17),      # threshold 0: phase 2 adds nothing
    (96, 16, 2, 7, 3.0, 4096),     # one full LDS sort, loose threshold
    (128, 32, 2, 20, 5.0, 10000),  # the reference's default rerank_m: up to three sorted runs placed by rank
    (96, 16, 0, 10, 1.0, 5000),    # every vector passes: two runs, repeated pool selects
]


@pytest.mark.parametrize("tp_screen", [1, 2])  # phase 1 in the two-phase kernel / through the MFMA screen
@pytest.mark.parametrize("dim,m,p1,limit_k,coeff,rerank_m", CASES)
def test_two_phase_bit_exact(dim, m, p1, limit_k, coeff, rerank_m, tp_screen):
    _say(f"two_phase dim={dim} m={m} p1={p1} limit_k={limit_k} coeff={coeff} rerank_m={rerank_m} "
         f"tp_screen={tp_screen}")
    rng = np.random.default_rng(dim + m + p1 + limit_k + rerank_m)
    nlist = 40
    offs, ids, lc, cent, cb = _index(rng, 30000, dim, m, nlist, empty=(3, 17), big=8)
    q = (rng.standard_normal((120, dim)) * 0.7).astype(np.float32)
    probes, _ = oracle.coarse(q, cent, 16)
    probes[5, 1] = 0xFFFFFFFF            # pruned probe (phase 1 when p1 > 1)
    probes[6, :] = 0xFFFFFFFF            # nothing probed: zero candidates
    probes[7, 0] = 3                     # an empty list first
    probes[8, 9] = 999                   # out-of-range id counts as pruned
    probes[9, 0] = 8                     # the long list (> 1024 vectors) in phase 1 ...
    probes[9, 12] = 8                    # ... and again in phase 2
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    idx.set_option(fg.Index.OPT_TWO_PHASE_SCREEN, tp_screen)
    assert idx.max_list_len > 1024
    gid, gd, gcnt, gcut, gthr = idx.two_phase_search(torch.from_numpy(q).cuda(),
                                                     torch.from_numpy(probes.view(np.int32)).cuda(), p1, limit_k,
                                                     coeff, rerank_m, want_cutoffs=True)
    gid, gd, gcnt, gthr = _host(gid), _host(gd), _host(gcnt), _host(gthr)
    oid, od, ocnt, ocut, othr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, coeff,
                                                        rerank_m)
    assert np.array_equal(gcnt, ocnt), np.nonzero(gcnt != ocnt)[0][:5]
    bad = np.nonzero(~np.all(gid == oid, axis=1))[0]
    assert bad.size == 0, f"first mismatching queries {bad[:5]}"
    assert np.array_equal(_bits(gd), _bits(od))
    assert np.array_equal(_bits(gthr), _bits(othr))
    if p1 > 0:
        assert np.array_equal(_bits(_host(gcut)), _bits(ocut))
    assert gcnt[6] == 0 and np.all(gid[6] == -1)
    # the count before the rerank_m cut (the reference's d_atomic); the results stay the same
    pid, pd, pcnt, _, _, pre = idx.two_phase_search(torch.from_numpy(q).cuda(),
                                                    torch.from_numpy(probes.view(np.int32)).cuda(), p1, limit_k,
                                                    coeff, rerank_m, want_pre_cut=True)
    *_, opre = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, coeff, rerank_m,
                                       want_pre_cut=True)
    assert np.array_equal(_host(pre), opre), np.nonzero(_host(pre) != opre)[0][:5]
    assert np.array_equal(_host(pid), oid) and np.array_equal(_bits(_host(pd)), _bits(od))
    assert np.array_equal(_host(pcnt), ocnt)
    idx.close()


@pytest.mark.parametrize("tp_screen", [1, 2])
def test_two_phase_many_phase1_lists(tp_screen):
    """More phase-1 lists than the kernel stages at once (16): the staged
    wave lists are merged in several rounds; unusable probes inside phase 1.
    Through the screen: more phase-1 lists than the one-wave final sorts, so
    every query takes the two-phase kernel's second half."""
    _say(f"two_phase p1=37 of nprobe=40 tp_screen={tp_screen}")
    rng = np.random.default_rng(4040)
    nlist = 64
    offs, ids, lc, cent, cb = _index(rng, 40000, 96, 32, nlist, empty=(5, 9, 30), big=12)
    q = (rng.standard_normal((90, 96)) * 0.7).astype(np.float32)
    probes, _ = oracle.coarse(q, cent, 40)
    probes[3, 7] = 0xFFFFFFFF
    probes[4, 20] = 5                    # an empty list inside phase 1
    probes[10, :17] = 0xFFFFFFFF         # exactly 20 usable phase-1 lists
    p1, limit_k, coeff, rerank_m = 37, 24, 1.1, 700
    idx = fg.Index.from_arrays(96, 32, offs, ids, lc, cent, cb)
    idx.set_option(fg.Index.OPT_TWO_PHASE_SCREEN, tp_screen)
    gid, gd, gcnt, gcut, gthr = idx.two_phase_search(torch.from_numpy(q).cuda(),
                                                     torch.from_numpy(probes.view(np.int32)).cuda(), p1, limit_k,
                                                     coeff, rerank_m, want_cutoffs=True)
    oid, od, ocnt, ocut, othr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, coeff,
                                                        rerank_m)
    assert np.array_equal(_host(gcnt), ocnt)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    assert np.array_equal(_bits(_host(gcut)), _bits(ocut))
    assert np.array_equal(_bits(_host(gthr)), _bits(othr))
    idx.close()


def test_two_phase_screen_phase1_short_lists_and_pruned_probes():
    """Phase 1 through the MFMA screen (limit_k <= 64): one single-probe
    query per (query, phase-1 probe).  Lists shorter than limit_k and probes
    without a list take their vectors directly, so nothing runs the LUT
    kernel; bit-exact with the oracle and with the LUT path (OPT_SCREEN 0)."""
    _say("two_phase screen phase 1: short lists, pruned probes")
    rng = np.random.default_rng(5151)
    dim, m, nlist = 96, 48, 64
    offs, ids, lc, cent, cb = _index(rng, 8000, dim, m, nlist, empty=(2, 11))
    lens = np.diff(offs)
    p1, limit_k, coeff, rerank_m = 12, 50, 1.0, 600
    short = np.nonzero((lens > 0) & (lens < limit_k))[0]
    assert short.size >= 3
    q = (rng.standard_normal((150, dim)) * 0.7).astype(np.float32)
    probes, _ = oracle.coarse(q, cent, 16)
    probes[4, :] = 0xFFFFFFFF            # nothing probed
    probes[5, 0] = short[0]              # a short list first
    probes[6, :3] = 0xFFFFFFFF           # pruned phase-1 probes
    probes[7, 1] = 2                     # an empty list in phase 1
    probes[8, 2] = 777                   # out of range: pruned
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    assert idx.screen_ready
    idx.set_option(fg.Index.OPT_TWO_PHASE_SCREEN, 2)  # 150 queries: below the automatic batch size
    dq, dp = torch.from_numpy(q).cuda(), torch.from_numpy(probes.view(np.int32)).cuda()
    gid, gd, gcnt, st = idx.two_phase_stats(dq, dp, p1, limit_k, coeff, rerank_m)
    oid, od, ocnt, _, _ = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, coeff, rerank_m)
    assert np.array_equal(_host(gcnt), ocnt)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    assert st["screen_virtual_queries"] == 150 * p1
    assert st["screen_no_threshold"] == 0
    assert st["screen_to_lut"] == st["screen_over_cap"]
    usable = (probes[:, :p1] < nlist) & (lens[np.minimum(probes[:, :p1], nlist - 1)] > 0)
    assert st["screen_candidates"] >= int(np.minimum(lens[probes[:, :p1][usable]], limit_k).sum())
    idx.set_option(fg.Index.OPT_SCREEN, 0)
    lid, ld, lcnt, _, _ = idx.two_phase_search(dq, dp, p1, limit_k, coeff, rerank_m)
    _, _, _, lst = idx.two_phase_stats(dq, dp, p1, limit_k, coeff, rerank_m)
    assert lst["screen_virtual_queries"] == 0
    assert np.array_equal(_host(lid), oid) and np.array_equal(_bits(_host(ld)), _bits(od))
    assert np.array_equal(_host(lcnt), ocnt)
    idx.close()


@pytest.mark.parametrize("dim,m,p1,limit_k,coeff,rerank_m", [
    (128, 32, 12, 50, 1.0, 1000),  # the reference pipeline's defaults (p1 12, limit_k 50)
    (96, 16, 5, 64, 1.2, 300),     # limit_k at the split's limit
    (128, 16, 2, 1, 1.0, 40),      # two phase-1 lists, one candidate each
])
def test_two_phase_split_phase1_equals_one_workgroup(dim, m, p1, limit_k, coeff, rerank_m):
    """Phase 1 spread over several workgroups a query (small batches) gives
    the one-workgroup result bit for bit, also with more workgroups than
    usable phase-1 lists; one split against the oracle."""
    _say(f"two_phase split dim={dim} m={m} p1={p1} limit_k={limit_k}")
    rng = np.random.default_rng(9000 + dim + m + p1)
    nlist = 48
    offs, ids, lc, cent, cb = _index(rng, 30000, dim, m, nlist, empty=(2, 11), big=6)
    q = (rng.standard_normal((60, dim)) * 0.7).astype(np.float32)
    probes, _ = oracle.coarse(q, cent, 16)
    probes[1, 0] = 2                     # an empty list first
    probes[2, :p1] = 0xFFFFFFFF          # no usable phase-1 list
    probes[3, 1] = 0xFFFFFFFF            # a pruned probe inside phase 1
    probes[4, 0] = 6                     # the long list in phase 1
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    dq, dp = torch.from_numpy(q).cuda(), torch.from_numpy(probes.view(np.int32)).cuda()
    outs = {}
    for split in (1, 2, 3, 7, 64):
        idx.set_option(fg.Index.OPT_TWO_PHASE_SPLIT, split)
        gid, gd, gcnt, gcut, gthr = idx.two_phase_search(dq, dp, p1, limit_k, coeff, rerank_m, want_cutoffs=True)
        outs[split] = (_host(gid), _bits(_host(gd)), _host(gcnt), _bits(_host(gcut)), _bits(_host(gthr)))
    idx.set_option(fg.Index.OPT_TWO_PHASE_SPLIT, 0)
    for split in (2, 3, 7, 64):
        for a, b in zip(outs[1], outs[split]):
            assert np.array_equal(a, b), f"split {split} differs"
    oid, od, ocnt, ocut, othr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, coeff,
                                                        rerank_m)
    gid, gd, gcnt, gcut, gthr = outs[7]
    assert np.array_equal(gcnt, ocnt)
    assert np.array_equal(gid, oid)
    assert np.array_equal(gd, _bits(od))
    assert np.array_equal(gcut, _bits(ocut))
    assert np.array_equal(gthr, _bits(othr))
    idx.close()


def test_two_phase_workspace_chunks_equal_one_launch():
    _say("two_phase chunked workspace")
    rng = np.random.default_rng(77)
    offs, ids, lc, cent, cb = _index(rng, 20000, 128, 32, 30)
    q = torch.from_numpy((rng.standard_normal((300, 128)) * 0.7).astype(np.float32)).cuda()
    idx = fg.Index.from_arrays(128, 32, offs, ids, lc, cent, cb)
    probes, _ = idx.coarse_search(q, 12)
    full = idx.two_phase_search(q, probes, 4, 20, 1.0, 200)
    one = fg.lib.fgpu_two_phase_workspace_bytes(1, 12, 4, 20, 200)
    small = torch.empty(one * 7 + 100, dtype=torch.uint8, device="cuda")   # 7 queries per launch
    part = idx.two_phase_search(q, probes, 4, 20, 1.0, 200, workspace=small)
    for a, b in zip(full[:3], part[:3]):
        assert torch.equal(a, b)
    idx.close()


# (dim, k, mb, eps, beta)
RERANK = [(96, 100, 128, 0.1, 2), (128, 10, 128, 0.1, 2), (96, 256, 32, -1.0, 2), (128, 20, 7, 0.5, 3),
          (128, 5, 16, 1.0, 1)]


@pytest.mark.parametrize("spec", [1, 4])
@pytest.mark.parametrize("dim,k,mb,eps,beta", RERANK)
def test_rerank_bit_exact(dim, k, mb, eps, beta, spec):
    """spec: mini-batches the kernel computes at once before applying them in
    order (4 is the default for batches that leave CUs free)."""
    _say(f"rerank dim={dim} k={k} mb={mb} eps={eps} beta={beta} spec={spec}")
    rng = np.random.default_rng(dim + k + mb)
    n, nq, rm = 20000, 200, 600
    base = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((nq, dim)).astype(np.float32)
    # candidates in a noisy "ADC" order: the exact ranking perturbed
    cand = np.empty((nq, rm), np.int32)
    for i in range(nq):
        pool = rng.choice(n, 3 * rm, replace=False)
        d = ((base[pool] - q[i]) ** 2).sum(1) * rng.uniform(0.7, 1.3, pool.size)
        cand[i] = pool[np.argsort(d)[:rm]]
    cand[3, 10] = -1                     # invalid ids are skipped
    cand[3, 11] = n + 5
    cand[4, 20] = cand[4, 2]             # a duplicate candidate
    counts = rng.integers(0, rm + 1, nq).astype(np.int32)
    counts[:6] = [rm, rm, 0, rm, rm, 1]
    gid, gd, gvis, gst, gfin = fg.rerank(torch.from_numpy(q).cuda(), torch.from_numpy(base).cuda(),
                                         torch.from_numpy(cand).cuda(), torch.from_numpy(counts).cuda(), k, mb, eps,
                                         beta, spec=spec, want_state=True)
    torch.cuda.synchronize()
    oid, od, ovis, ost, ofin = oracle.rerank(q, base, cand, counts, k, mb, eps, beta, want_state=True)
    gid, gd, gvis = _host(gid), _host(gd), _host(gvis)
    assert np.array_equal(gvis, ovis), np.nonzero(gvis != ovis)[0][:5]
    assert np.array_equal(_host(gst), ost) and np.array_equal(_host(gfin), ofin)
    bad = np.nonzero(~np.all(gid == oid, axis=1))[0]
    assert bad.size == 0, f"first mismatching queries {bad[:5]}"
    assert np.array_equal(_bits(gd), _bits(od))
    assert np.all(gid[2] == -1)


@pytest.mark.parametrize("tp_screen", [1, 2])
def test_search_rerank_end_to_end(tp_screen):
    """Coarse + two-phase + rerank; through the screen the phase-2 list bounds
    come from the coarse step's probe distances."""
    _say(f"search_rerank end to end tp_screen={tp_screen}")
    x = oracle.gen_gmm(30000, 96, 48, seed=11, sig_lo=0.05, sig_hi=0.15)
    q = oracle.gen_gmm(300, 96, 48, seed=11, set=1, sig_lo=0.05, sig_hi=0.15)
    offs, ids, codes, cent, cb = fg.build_ivfpq(torch.from_numpy(x).cuda(), 64, 48, kmeans_iters=4, init_mode=1,
                                                seed=3, pq_iters=3, sample_size=5000)
    idx = fg.Index.from_arrays(96, 48, offs, ids, codes, cent, cb)
    idx.set_option(fg.Index.OPT_TWO_PHASE_SCREEN, tp_screen)
    dq, dx = torch.from_numpy(q).cuda(), torch.from_numpy(x).cuda()
    gid, gd = idx.search_rerank(dq, dx, 16, 20, p1_lists=4, limit_k=30, threshold_coeff=1.0, rerank_m=200)
    probes, _ = oracle.coarse(q, cent, 16)
    tid, td, tc, _, _ = oracle.search_two_phase(q, cent, cb, offs, ids, codes, probes, 4, 30, 1.0, 200)
    oid, od, _ = oracle.rerank(q, x, tid, tc, 20, 128, 0.1, 2)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    idx.close()


@pytest.mark.parametrize("limit_k,p1,rerank_m", [(65, 12, 1000), (300, 6, 2500), (4096, 4, 20000)])
def test_two_phase_large_limit_k(limit_k, p1, rerank_m):
    """limit_k above 64 (the reference's tuner sets it to the largest rank of
    a true neighbour in its list): each phase-1 list's keys are cut to its
    limit_k best in the pool.  Lists longer than 2048 (several segments and
    selects), lists shorter than limit_k (w = n), a list probed twice."""
    _say(f"two_phase limit_k={limit_k} p1={p1} rerank_m={rerank_m}")
    rng = np.random.default_rng(limit_k)
    nlist = 30
    offs, ids, lc, cent, cb = _index(rng, 45000, 96, 32, nlist, empty=(4,), big=7)
    assert np.diff(offs).max() > 4096
    q = (rng.standard_normal((60, 96)) * 0.7).astype(np.float32)
    probes, _ = oracle.coarse(q, cent, 10)
    probes[1, 0] = 7                     # the long list first ...
    probes[1, 1] = 7                     # ... and again
    probes[2, 0] = 4                     # an empty list in phase 1
    probes[3, 2] = 0xFFFFFFFF
    idx = fg.Index.from_arrays(96, 32, offs, ids, lc, cent, cb)
    gid, gd, gcnt, gcut, gthr = idx.two_phase_search(torch.from_numpy(q).cuda(),
                                                     torch.from_numpy(probes.view(np.int32)).cuda(), p1, limit_k,
                                                     1.0, rerank_m, want_cutoffs=True)
    oid, od, ocnt, ocut, othr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, 1.0,
                                                        rerank_m)
    assert np.array_equal(_host(gcnt), ocnt)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    assert np.array_equal(_bits(_host(gcut)), _bits(ocut))
    assert np.array_equal(_bits(_host(gthr)), _bits(othr))
    idx.close()


def test_two_phase_many_probes():
    """nprobe 200 with 70 phase-1 lists (both above one 64-probe chunk): probe
    compaction over four chunks, cutoffs past index 64, pruned and empty
    probes in the later chunks."""
    _say("two_phase nprobe=200 p1=70")
    rng = np.random.default_rng(2200)
    nlist = 300
    offs, ids, lc, cent, cb = _index(rng, 60000, 96, 48, nlist, empty=(5, 77, 150), big=20)
    q = (rng.standard_normal((80, 96)) * 0.7).astype(np.float32)
    probes, _ = oracle.coarse(q, cent, 200)
    probes[2, 66] = 0xFFFFFFFF           # pruned inside phase 1, second chunk
    probes[3, 130] = 0xFFFFFFFF          # pruned in phase 2, third chunk
    probes[4, 199] = 150                 # empty list in the last chunk
    probes[5, 65] = 77                   # empty list in phase 1, second chunk
    p1, limit_k, coeff, rerank_m = 70, 20, 1.2, 2000
    idx = fg.Index.from_arrays(96, 48, offs, ids, lc, cent, cb)
    gid, gd, gcnt, gcut, gthr = idx.two_phase_search(torch.from_numpy(q).cuda(),
                                                     torch.from_numpy(probes.view(np.int32)).cuda(), p1, limit_k,
                                                     coeff, rerank_m, want_cutoffs=True)
    oid, od, ocnt, ocut, othr = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, coeff,
                                                        rerank_m)
    assert np.array_equal(_host(gcnt), ocnt)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    assert np.array_equal(_bits(_host(gcut)), _bits(ocut))
    assert np.array_equal(_bits(_host(gthr)), _bits(othr))
    assert np.all(_host(gcut)[:, 64:] >= 0) and (_host(gcut)[:, 64:] > 0).any()
    idx.close()


def test_search_rerank_many_probes():
    """The whole general search at nprobe 128 (coarse top-128, two-phase,
    rerank) against the oracle."""
    _say("search_rerank nprobe=128")
    x = oracle.gen_gmm(40000, 96, 64, seed=12, sig_lo=0.05, sig_hi=0.15)
    q = oracle.gen_gmm(200, 96, 64, seed=12, set=1, sig_lo=0.05, sig_hi=0.15)
    offs, ids, codes, cent, cb = fg.build_ivfpq(torch.from_numpy(x).cuda(), 256, 48, kmeans_iters=4, init_mode=1,
                                                seed=3, pq_iters=3, sample_size=5000)
    idx = fg.Index.from_arrays(96, 48, offs, ids, codes, cent, cb)
    dq, dx = torch.from_numpy(q).cuda(), torch.from_numpy(x).cuda()
    gid, gd = idx.search_rerank(dq, dx, 128, 20, p1_lists=80, limit_k=30, threshold_coeff=1.0, rerank_m=600)
    probes, _ = oracle.coarse(q, cent, 128)
    assert (probes[:, 64:] != 0xFFFFFFFF).any()
    tid, td, tc, _, _ = oracle.search_two_phase(q, cent, cb, offs, ids, codes, probes, 80, 30, 1.0, 600)
    oid, od, _ = oracle.rerank(q, x, tid, tc, 20, 128, 0.1, 2)
    assert np.array_equal(_host(gid), oid)
    assert np.array_equal(_bits(_host(gd)), _bits(od))
    idx.close()


def test_build_ivfpq_sampled_bit_exact():
    _say("build_ivfpq sampled k-means training")
    x = oracle.gen_gmm(9000, 96, 16, seed=4, sig_lo=0.05, sig_hi=0.15)
    got = fg.build_ivfpq(torch.from_numpy(x).cuda(), 24, 48, kmeans_iters=3, init_mode=1, seed=5, pq_iters=2,
                         sample_size=2000, train_rows=2500)
    want = oracle.build_ivfpq(x, 24, 48, kmeans_iters=3, init_mode=1, seed=5, pq_iters=2, sample_size=2000,
                              train_rows=2500)
    for g, w, name in zip(got, want, ["offsets", "ids", "codes", "centroids", "codebook"]):
        assert np.array_equal(np.asarray(g).view(np.uint8), np.asarray(w).view(np.uint8)), name


@pytest.mark.parametrize("k,n,dim", [(10, 10000, 96), (100, 9000, 128), (128, 4097, 96), (1, 5000, 64),
                                     (64, 50, 128)])
def test_knn_exact_bit_exact(k, n, dim):
    _say(f"knn_exact k={k} n={n} dim={dim}")
    rng = np.random.default_rng(k + n + dim)
    base = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((150, dim)).astype(np.float32)
    base[min(4099, n - 1)] = base[7]      # a duplicate row in a later chunk: the lower id wins the tie
    q[0] = base[7]                        # distance exactly 0 to both
    q[1] = base[n - 1] + np.float32(1e-3)
    gid, gd = fg.knn_exact(torch.from_numpy(q).cuda(), torch.from_numpy(base).cuda(), k)
    oid, od = oracle.knn_exact(q, base, k)
    gid, gd = _host(gid), _host(gd)
    bad = np.nonzero(~np.all(gid == oid, axis=1))[0]
    assert bad.size == 0, f"first mismatching queries {bad[:5]}: gpu {gid[bad[0]][:8]} oracle {oid[bad[0]][:8]}"
    assert np.array_equal(_bits(gd), _bits(od))
    if n < k:
        assert np.all(gid[:, n:] == -1)


def test_reference_default_rerank_m_end_to_end():
    """The reference's default rerank_m = 10000 (defs.h:18) through the
    two-phase scan and the exact rerank, against the oracle."""
    _say("two_phase + rerank with rerank_m 10000")
    rng = np.random.default_rng(10000)
    dim, m, nlist, k = 128, 32, 48, 10
    offs, ids, lc, cent, cb = _index(rng, 40000, dim, m, nlist, big=4)
    base = (rng.standard_normal((40000, dim)) * 0.7).astype(np.float32)
    q = (rng.standard_normal((64, dim)) * 0.7).astype(np.float32)
    probes, _ = oracle.coarse(q, cent, 20)
    p1, limit_k, coeff, rerank_m = 12, 50, 2.5, 10000
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    dq = torch.from_numpy(q).cuda()
    tid, td, tc, _, _ = idx.two_phase_search(dq, torch.from_numpy(probes.view(np.int32)).cuda(), p1, limit_k, coeff,
                                             rerank_m)
    oid, od, ocnt, _, _ = oracle.search_two_phase(q, cent, cb, offs, ids, lc, probes, p1, limit_k, coeff, rerank_m)
    assert np.array_equal(_host(tc), ocnt)
    assert (ocnt > 4096).any(), "the case must need more than one LDS sort"
    assert np.array_equal(_host(tid), oid) and np.array_equal(_bits(_host(td)), _bits(od))
    rid, rd, vis = fg.rerank(dq, torch.from_numpy(base).cuda(), tid, tc, k, 128, 0.1, 2)
    fid, fd, fvis = oracle.rerank(q, base, oid, ocnt, k, 128, 0.1, 2)
    assert np.array_equal(_host(rid), fid) and np.array_equal(_bits(_host(rd)), _bits(fd))
    assert np.array_equal(_host(vis), fvis)
    idx.close()
