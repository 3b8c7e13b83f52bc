"""The plain search under HIP graph capture: fgpu_search with a caller
workspace (and fgpu_search_noalloc) enqueue kernels only -- no allocation,
memset or host synchronisation -- so a serving loop can capture a batch once
and replay it.  Each replay is checked against the eager result, with eager
calls between the replays."""
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


@pytest.mark.parametrize("noalloc,captured_first", [(False, False), (True, False), (True, True), (False, True)])
def test_search_replays_from_a_graph(noalloc, captured_first):
    """captured_first: the index's first search is the captured one (index
    creation has made every per-device lookup a search needs)."""
    _say(f"graph capture of the plain search (noalloc={noalloc}, first call captured={captured_first})")
    rng = np.random.default_rng(99)
    dim, m, nlist, nq, nprobe, k = 128, 32, 200, 3000, 24, 10
    x = oracle.gen_gmm(60000, dim, 40, seed=9, sig_lo=0.08)
    q = oracle.gen_gmm(nq, dim, 40, seed=9, set=1, sig_lo=0.08)
    offs, ids, codes, cent, cb = fg.build_ivfpq(torch.from_numpy(x).cuda(), nlist, m, kmeans_iters=4, init_mode=1,
                                                seed=3, pq_iters=3, sample_size=5000)
    idx = fg.Index.from_arrays(dim, m, offs, ids, codes, cent, cb)
    dq = torch.from_numpy(q).cuda()
    oi = torch.empty((nq, k), dtype=torch.int32, device="cuda")
    od = torch.empty((nq, k), dtype=torch.float32, device="cuda")
    if noalloc:
        step = lambda: idx.search_noalloc(dq, nprobe, k, out=(oi, od))  # noqa: E731
    else:
        ws = torch.empty(idx.search_workspace_bytes(nq, nprobe), dtype=torch.uint8, device="cuda")
        step = lambda: idx.search(dq, nprobe, k, workspace=ws, out=(oi, od))  # noqa: E731
    g = torch.cuda.CUDAGraph()
    if captured_first:
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            step()
        torch.cuda.synchronize()
    step()
    torch.cuda.synchronize()
    ref_i, ref_d = oi.clone(), od.clone()
    probes, _ = oracle.coarse(q[:200], cent, nprobe)
    wid, wd = oracle.search_plain(q[:200], cent, cb, offs, ids, codes, probes, k)
    assert np.array_equal(ref_i[:200].cpu().numpy(), wid)
    if not captured_first:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            step()
        torch.cuda.synchronize()
    for _ in range(4):
        oi.fill_(-7)
        od.fill_(-1.0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(oi, ref_i)
        assert torch.equal(od.view(torch.int32), ref_d.view(torch.int32))
        step()  # eager work between the replays
        torch.cuda.synchronize()
    assert idx.faults() == 0
    idx.close()
