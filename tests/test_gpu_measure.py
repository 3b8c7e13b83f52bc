"""The measurement probes read what they claim: the XOR of every 32-bit word
the streaming read and the random-row gather load, folded over their sink,
equals the same XOR computed on the host."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():
    pytest.skip("no HIP device", allow_module_level=True)

import fusiongpu_amd as fg  # noqa: E402


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def _fold(sink):
    v = sink.cpu().numpy().view(np.uint64)
    return int(np.bitwise_xor.reduce(v.astype(np.uint64) & np.uint64(0xFFFFFFFF)))


def test_stream_read_reads_every_word():
    _say("stream_read XOR check")
    rng = np.random.default_rng(1)
    a = rng.integers(0, 2**32, size=(3 << 20) // 4 + 12, dtype=np.uint32)  # not a multiple of the grid stride
    d = torch.from_numpy(a.view(np.int32)).cuda()
    sink = torch.zeros(fg.lib.fgpu_stream_read_grid(), dtype=torch.int64, device="cuda")
    fg._check(fg.lib.fgpu_stream_read(d.data_ptr(), d.numel() * 4, sink.data_ptr(), None))
    torch.cuda.synchronize()
    assert _fold(sink) == int(np.bitwise_xor.reduce(a))


@pytest.mark.parametrize("lanes", [1, 8])
@pytest.mark.parametrize("dim", [96, 128])
def test_row_gather_reads_the_indexed_rows(dim, lanes):
    _say(f"row_gather XOR check, {dim * 4}-byte rows, {lanes} lanes a row")
    rng = np.random.default_rng(dim)
    rows = rng.integers(0, 2**32, size=(5000, dim), dtype=np.uint32)
    idx = rng.integers(0, 5000, size=77777).astype(np.int32)  # not a multiple of the rows a workgroup reads
    d = torch.from_numpy(rows.view(np.float32)).cuda()
    di = torch.from_numpy(idx).cuda()
    sink = torch.zeros(fg.lib.fgpu_stream_read_grid(), dtype=torch.int64, device="cuda")
    fg._check(fg.lib.fgpu_row_gather_lanes(d.data_ptr(), 5000, dim * 4, di.data_ptr(), idx.size, lanes,
                                           sink.data_ptr(), None))
    torch.cuda.synchronize()
    per_row = np.bitwise_xor.reduce(rows, axis=1)
    assert _fold(sink) == int(np.bitwise_xor.reduce(per_row[idx]))
    if lanes == 8:  # fgpu_row_gather is the eight-lane form
        sink.zero_()
        fg._check(fg.lib.fgpu_row_gather(d.data_ptr(), 5000, dim * 4, di.data_ptr(), idx.size, sink.data_ptr(), None))
        torch.cuda.synchronize()
        assert _fold(sink) == int(np.bitwise_xor.reduce(per_row[idx]))
    fg.row_gather(d, di, lanes_per_row=lanes)  # the Python wrapper runs the same call
    torch.cuda.synchronize()


def test_row_gather_rejects_other_lane_counts():
    d = torch.zeros(16, 96, device="cuda")
    di = torch.zeros(4, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="lanes_per_row"):
        fg.row_gather(d, di, lanes_per_row=4)
