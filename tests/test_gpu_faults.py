"""The scan kernel's bounded waits: a give-up is counted on the index and marks
the results it may have touched, never leaving silently wrong ids.

Give-ups are forced from the host only (the index's FGPU_OPT_SPIN_LIMIT): every
wave still runs to the end of the kernel, and the kernel clamps every list
range it reads from LDS to the index, so its loads stay in bounds whatever
the hand-off counters say.
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


def _index(rng, n, dim, m, nlist, p=None):
    p = rng.random(nlist) + 0.05 if p is None else p
    assign = rng.choice(nlist, size=n, p=p / p.sum()).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = rng.standard_normal((nlist, dim)).astype(np.float32) * 0.7
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    return offs, ids, lc, cent, cb


def test_forced_give_ups_are_counted_and_mark_results():
    _say("faults: spin limit 1 (forced give-ups), then the automatic limit")
    rng = np.random.default_rng(71)
    dim, m, nlist, nq, k = 128, 32, 48, 2000, 10
    offs, ids, lc, cent, cb = _index(rng, 40000, dim, m, nlist)
    q = rng.standard_normal((nq, dim)).astype(np.float32) * 0.7
    probes, pdist = oracle.coarse(q, cent, 12)
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, k)
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    dq, dp, dpd = (torch.from_numpy(q).cuda(), torch.from_numpy(probes.view(np.int32)).cuda(),
                   torch.from_numpy(pdist).cuda())
    assert idx.faults() == 0
    idx.set_option(fg.Index.OPT_SPIN_LIMIT, 1)
    gid, gd = idx.adc_search(dq, dp, k, probe_dists=dpd)
    gid, gd = gid.cpu().numpy(), gd.cpu().numpy()
    nf = idx.faults()
    idx.set_option(fg.Index.OPT_SPIN_LIMIT, 0)
    assert nf > 0, "a poll limit of 1 must make waits give up"
    with pytest.raises(fg.FgpuError) as e:
        idx.check()
    assert e.value.status == 7
    marked = np.all(gid == fg.FAULT_ID, axis=1)
    assert marked.any()
    # every row is either marked in all slots (ids -2, NaN distances) or exact
    assert np.isnan(gd[marked]).all()
    rest = ~marked
    assert np.array_equal(gid[rest], oid[rest])
    assert np.array_equal(gd[rest].view(np.uint32), od[rest].view(np.uint32))
    assert not np.any(gid[rest] == fg.FAULT_ID)
    # reset, then the automatic limit: exact and no give-up
    assert idx.faults(reset=True) == nf
    assert idx.faults() == 0
    gid, gd = idx.adc_search(dq, dp, k, probe_dists=dpd)
    assert np.array_equal(gid.cpu().numpy(), oid)
    assert np.array_equal(gd.cpu().numpy().view(np.uint32), od.view(np.uint32))
    idx.check()
    idx.close()


def test_forced_give_ups_with_dynamic_query_claims():
    """search on the LUT kernels (coarse, then the flow scan with queries
    claimed from a counter): rows a give-up kept from completing keep the
    marker written at set-up; another index is unaffected by the option."""
    _say("faults: dynamic claims, spin limit 1")
    rng = np.random.default_rng(73)
    dim, m, nlist, nq, k = 128, 32, 48, 3000, 10
    offs, ids, lc, cent, cb = _index(rng, 40000, dim, m, nlist)
    q = rng.standard_normal((nq, dim)).astype(np.float32) * 0.7
    probes, _ = oracle.coarse(q, cent, 12)
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, k)
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    idx.set_option(fg.Index.OPT_SCREEN, 0)  # the LUT flow kernel, whose waits this test forces to give up
    dq = torch.from_numpy(q).cuda()
    idx.set_option(fg.Index.OPT_SPIN_LIMIT, 1)
    gid, gd = idx.search(dq, 12, k)
    gid, gd = gid.cpu().numpy(), gd.cpu().numpy()
    nf = idx.faults(reset=True)
    idx.set_option(fg.Index.OPT_SPIN_LIMIT, 0)
    assert nf > 0
    marked = np.all(gid == fg.FAULT_ID, axis=1)
    assert marked.any()
    assert np.isnan(gd[marked]).all()
    rest = ~marked
    assert np.array_equal(gid[rest], oid[rest])
    assert np.array_equal(gd[rest].view(np.uint32), od[rest].view(np.uint32))
    gid, gd = idx.search(dq, 12, k)
    assert np.array_equal(gid.cpu().numpy(), oid)
    assert np.array_equal(gd.cpu().numpy().view(np.uint32), od.view(np.uint32))
    idx.check()
    # The option belongs to its index: a second index over the same arrays
    # keeps the automatic limit while the first one forces give-ups.
    other = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    other.set_option(fg.Index.OPT_SCREEN, 0)
    idx.set_option(fg.Index.OPT_SPIN_LIMIT, 1)
    gid, gd = other.search(dq, 12, k)
    assert np.array_equal(gid.cpu().numpy(), oid)
    assert np.array_equal(gd.cpu().numpy().view(np.uint32), od.view(np.uint32))
    assert other.faults() == 0
    other.close()
    idx.close()


def test_one_very_long_list_within_the_automatic_limit():
    """A list of 300k vectors (the flow kernel's waits then last a whole list
    scan) next to short ones: exact, and no wait gives up."""
    _say("faults: one 300k-vector list")
    rng = np.random.default_rng(72)
    dim, m, nlist, nq, k = 128, 32, 16, 600, 10
    p = np.full(nlist, 0.02)
    p[3] = 10.0
    offs, ids, lc, cent, cb = _index(rng, 320000, dim, m, nlist, p)
    assert np.diff(offs).max() > 290000
    q = rng.standard_normal((nq, dim)).astype(np.float32) * 0.7
    probes, pdist = oracle.coarse(q, cent, 4)
    probes[:, 0] = 3  # every query scans the long list first
    pdist[:, 0] = oracle.coarse(q, cent[3:4], 1)[1][:, 0]
    oid, od = oracle.search_plain(q, cent, cb, offs, ids, lc, probes, k)
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    gid, gd = idx.adc_search(torch.from_numpy(q).cuda(), torch.from_numpy(probes.view(np.int32)).cuda(), k,
                             probe_dists=torch.from_numpy(pdist).cuda())
    assert np.array_equal(gid.cpu().numpy(), oid)
    assert np.array_equal(gd.cpu().numpy().view(np.uint32), od.view(np.uint32))
    assert idx.faults() == 0
    idx.close()
