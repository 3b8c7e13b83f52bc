"""The Python mirror's argument handling, on the CPU: dtype conversion and
shape checks before anything reaches the C ABI, and the stream scope every
device call runs in."""
import contextlib

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import fusiongpu_amd as fg  # noqa: E402


def test_arg_converts_the_dtypes_the_abi_reads():
    a = fg._arg(np.ones((3, 4), np.float64), torch.float32, "x", (None, 4))
    assert a.dtype == torch.float32 and tuple(a.shape) == (3, 4)
    # int64 probe ids convert; 0xFFFFFFFF, the pruned sentinel, stays all-ones
    p = fg._arg(np.array([[0, 5, 0xFFFFFFFF]], np.int64), torch.int32, "probe_ids", (1, None))
    assert p.dtype == torch.int32
    assert p.numpy().view(np.uint32).tolist() == [[0, 5, 0xFFFFFFFF]]
    t = torch.arange(6, dtype=torch.int64).reshape(2, 3)
    assert fg._arg(t, torch.int32, "ids").dtype == torch.int32
    assert fg._arg(np.array([-1, (1 << 31) - 1, -(1 << 31)], np.int64), torch.int32, "ids").tolist() \
        == [-1, (1 << 31) - 1, -(1 << 31)]


@pytest.mark.parametrize("v", [1 << 31, (1 << 32) + 3, -(1 << 31) - 1, 1 << 40])
def test_arg_rejects_ids_that_do_not_fit_int32(v):
    with pytest.raises(ValueError, match="does not fit in int32"):
        fg._arg(np.array([[0, v]], np.int64), torch.int32, "ids")
    with pytest.raises(ValueError, match="does not fit in int32"):
        fg._arg(torch.tensor([7, v], dtype=torch.int64), torch.int32, "ids")


@pytest.mark.parametrize("bad,dtype", [(np.ones((2, 4), np.int32), torch.float32),
                                       (np.ones((2, 4), np.float32), torch.int32),
                                       (np.ones((2, 4), np.complex64), torch.float32),
                                       (np.ones((2, 4), bool), torch.int32)])
def test_arg_rejects_unreadable_dtypes(bad, dtype):
    with pytest.raises(TypeError):
        fg._arg(bad, dtype, "x")


def test_arg_rejects_wrong_shapes():
    with pytest.raises(ValueError, match="dimension 1 is 64, expected 128"):
        fg._arg(np.zeros((5, 64), np.float32), torch.float32, "queries", (None, 128))
    with pytest.raises(ValueError, match="expected 2 dimensions"):
        fg._arg(np.zeros(128, np.float32), torch.float32, "queries", (None, 128))
    with pytest.raises(ValueError, match="dimension 0 is 4, expected 5"):
        fg._arg(np.zeros((4, 8), np.int32), torch.int32, "probe_ids", (5, None))
    with pytest.raises(TypeError):
        fg._arg([[1.0, 2.0]], torch.float32, "queries")


def test_out_checks_dtype_shape_and_device():
    with pytest.raises(ValueError):
        fg._out(torch.empty((3, 10), dtype=torch.int64), torch.int32, (3, 10), "out")
    with pytest.raises(ValueError):
        fg._out(torch.empty((3, 9), dtype=torch.int32), torch.int32, (3, 10), "out")
    with pytest.raises(ValueError):  # host memory is not device memory
        fg._out(torch.empty((3, 10), dtype=torch.int32), torch.int32, (3, 10), "out")


def _stub_index():
    idx = fg.Index.__new__(fg.Index)
    idx._h = None
    idx.dim, idx.pq_m, idx.nlist, idx.total, idx.max_list_len = 128, 32, 64, 1000, 40
    return idx


def test_index_methods_check_query_width_first():
    idx = _stub_index()
    q = np.zeros((5, 64), np.float32)
    for call in (lambda: idx.search(q, 8, 10), lambda: idx.coarse_search(q, 8),
                 lambda: idx.adc_search(q, np.zeros((5, 8), np.int32), 10),
                 lambda: idx.two_phase_search(q, np.zeros((5, 8), np.int32), 4, 10, 1.0, 100),
                 lambda: idx.search_rerank(q, np.zeros((10, 128), np.float32), 8, 10)):
        with pytest.raises(ValueError, match="queries"):
            call()
    with pytest.raises(TypeError):
        idx.search(np.zeros((5, 128), np.int32), 8, 10)


class _Sentinel(Exception):
    pass


def test_every_device_call_runs_inside_the_callers_stream_scope(monkeypatch):
    """Internal tensors (workspace, temporaries, outputs) are allocated while
    the caller's stream is current, so the caching allocator ties them to the
    stream the kernels run on: entering the scope must come before the first
    argument is converted or anything is allocated."""
    events = []

    @contextlib.contextmanager
    def fake_on(stream):
        events.append(("enter", stream))
        try:
            yield
        finally:
            events.append(("exit", stream))

    def fake_dev(*a, **k):
        events.append(("dev",))
        raise _Sentinel()

    monkeypatch.setattr(fg, "_on", fake_on)
    monkeypatch.setattr(fg, "_dev", fake_dev)
    idx = _stub_index()
    s = object()
    q = np.zeros((5, 128), np.float32)
    calls = [
        lambda: idx.search(q, 8, 10, stream=s),
        lambda: idx.coarse_search(q, 8, stream=s),
        lambda: idx.adc_search(q, np.zeros((5, 8), np.int32), 10, stream=s),
        lambda: idx.adc_search_stats(q, np.zeros((5, 8), np.int32), 10, stream=s),
        lambda: idx.two_phase_search(q, np.zeros((5, 8), np.int32), 4, 10, 1.0, 100, stream=s),
        lambda: idx.two_phase_stats(q, np.zeros((5, 8), np.int32), 4, 10, 1.0, 100, stream=s),
        lambda: idx.search_rerank(q, q, 8, 10, stream=s),
        lambda: idx.coarse_graph_search(q, 8, np.zeros((64, 8), np.int32), stream=s),
        lambda: idx.tune_list_stats(q, np.zeros(3, np.int32), np.zeros(3, np.int32), stream=s),
        lambda: fg.probe_counts(idx, np.zeros((5, 8), np.int32), stream=s),
        lambda: fg.rerank(q, q, np.zeros((5, 8), np.int32), np.zeros(5, np.int32), 4, stream=s),
        lambda: fg.l2_topk(q, q, 1, stream=s),
        lambda: fg.knn_exact(q, q, 1, stream=s),
        lambda: fg.graph_search(q, q, np.zeros((5, 4), np.int32), 1, stream=s),
        lambda: fg.kmeans_update(q, np.zeros(5, np.int32), None, 0, stream=s),
        lambda: fg.kmeans_fit(q, 2, 1, stream=s),
        lambda: fg.pq_train(q, np.zeros(5, np.int32), q, 32, stream=s),
        lambda: fg.pq_encode(q, np.zeros(5, np.int32), q, q, stream=s),
        lambda: fg.build_ivfpq(q, 2, 32, stream=s),
    ]
    for i, call in enumerate(calls):
        events.clear()
        with pytest.raises(_Sentinel):
            call()
        assert events[:2] == [("enter", s), ("dev",)], f"call {i}: {events}"
        assert events[-1] == ("exit", s), f"call {i}: {events}"
