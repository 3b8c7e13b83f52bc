"""fgpu_search_noalloc: the plain search with its scratch in the library's
fixed per-GPU device array (no workspace, no allocation).  It must give
fgpu_search's results bit for bit, call after call; the second call is
smaller than the first, so stale contents of the shared array from the first
call must not leak into it."""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import fusiongpu_amd as fg  # noqa: E402
import oracle  # noqa: E402


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def test_noalloc_limits_on_the_host():
    assert fg.lib.fgpu_search_noalloc_max_bytes() == 32 << 20
    rows = fg.lib.fgpu_search_noalloc_max_rows(4096, 32)
    assert rows % 64 == 0 and rows >= 64
    assert fg.lib.fgpu_search_workspace_bytes(rows, 4096, 32) <= 32 << 20
    assert fg.lib.fgpu_search_workspace_bytes(rows + 64, 4096, 32) > 32 << 20
    assert fg.lib.fgpu_search_noalloc_max_rows(1024, 32) >= 1664   # C2 runs in seven chunks
    assert fg.lib.fgpu_search_noalloc_max_rows(200000, 32) == 0     # beyond the array: rejected


@pytest.mark.gpu
def test_search_noalloc_equals_search_on_consecutive_calls():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    _say("search_noalloc: nlist 4096 (several chunks), then a smaller call")
    rng = np.random.default_rng(81)
    dim, m, nlist, nprobe, k = 128, 32, 4096, 24, 10
    n = 120000
    assign = rng.integers(0, nlist, n).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = rng.standard_normal((nlist, dim)).astype(np.float32) * 0.7
    cb = (rng.standard_normal((m, 256, dim // m)) * 0.4).astype(np.float32)
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    rows = fg.lib.fgpu_search_noalloc_max_rows(nlist, nprobe)
    q = torch.from_numpy(rng.standard_normal((5000, dim)).astype(np.float32) * 0.7).cuda()
    assert q.shape[0] > 2 * rows  # at least three chunks
    for nq in (5000, 777):
        qq = q[:nq].contiguous()
        ref_id, ref_d = idx.search(qq, nprobe, k)
        out = (torch.full((nq, k), 123, dtype=torch.int32, device="cuda"),
               torch.full((nq, k), 5.0, dtype=torch.float32, device="cuda"))
        gid, gd = idx.search_noalloc(qq, nprobe, k, out=out)
        torch.cuda.synchronize()
        assert torch.equal(gid, ref_id) and torch.equal(gd, ref_d), f"nq {nq}: differs from fgpu_search"
    # and against the oracle, on the smaller call
    qn = q[:777].cpu().numpy()
    op, _ = oracle.coarse(qn, cent, nprobe)
    oid, od = oracle.search_plain(qn, cent, cb, offs, ids, lc, op, k)
    assert np.array_equal(gid.cpu().numpy(), oid)
    assert np.array_equal(gd.cpu().numpy().view(np.uint32), od.view(np.uint32))
    assert idx.faults() == 0
    idx.close()


@pytest.mark.gpu
def test_search_noalloc_rejects_an_index_beyond_the_array():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    rng = np.random.default_rng(82)
    dim, m, nlist = 32, 16, 140000
    n = 1000
    assign = rng.integers(0, nlist, n).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    offs, ids, lc = oracle.build_lists(assign, nlist, codes)
    cent = rng.standard_normal((nlist, dim)).astype(np.float32)
    cb = rng.standard_normal((m, 256, dim // m)).astype(np.float32)
    idx = fg.Index.from_arrays(dim, m, offs, ids, lc, cent, cb)
    q = torch.zeros((10, dim), dtype=torch.float32, device="cuda")
    with pytest.raises(fg.FgpuError) as e:
        idx.search_noalloc(q, 8, 10)
    assert e.value.status == 6 and "scratch" in str(e.value)
    idx.close()
