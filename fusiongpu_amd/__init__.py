"""fusiongpu_amd -- MI355X-native IVF-PQ search engine.

Python host mirror of the C ABI in include/fusiongpu.h (libfusiongpu.so).
Device buffers are torch tensors on the HIP device (torch is plumbing for
memory and streams); every compute call goes to the HIP kernels in
fusiongpu_amd/csrc.  There is no CPU fallback: importing this package raises
if the library is not built.

Reference interfaces mirrored (Hello-day/FusionGPU):
  * Index.load / Index.from_arrays  -> load_ivf_index_to_gpu (search_pipeline.cu:481-529)
  * Index.coarse_search             -> cuVS CAGRA top_m call (search_pipeline.cu:341)
  * Index.adc_search                -> run_gpu_batch_logic with p1_lists = nprobe,
                                       limit_k = rerank_m = k (gpu_global.cu:679-874)
  * Index.two_phase_search          -> run_gpu_batch_logic, general form (gpu_global.cu:679-874)
  * rerank                          -> run_gpu_rerank (gpu_global.cu:603-673)
  * Index.search_rerank             -> SearchPipeline::submit_batch's device path (search_pipeline.cu:341-361)
  * kmeans_fit / l2_topk            -> run_kmeans_gpu / batch_assign_clusters (kmeans_gpu.cuh:197-324)
  * knn_exact                       -> brute_force_search_kernel (tune_parameters.cu:49-96)
  * graph_search                    -> the cuVS CAGRA search role (cagra_adapter.cuh:38-68), own algorithm
  * pq_train                        -> train_residual_pq_codebooks (pq_utils.h:77-138)
  * pq_encode                       -> encode_residuals_to_pq_gpu (kmeans_gpu.cuh:450-508)
  * build_ivfpq                     -> build_global main (build_global.cu:21-258), no rebalancing
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import numpy as np

__all__ = [
    "FgpuError", "lib", "lib_path", "Index", "gen_gmm", "l2_topk", "kmeans_fit", "kmeans_update",
    "fixed_shift", "pq_train", "pq_encode", "build_ivfpq", "write_ivf_data", "read_ivf_data",
    "write_fvecs", "read_fvecs", "read_ivecs", "probe_counts", "rerank", "knn_exact", "graph_search",
    "stream_read", "row_gather", "FAULT_ID", "prune_probes", "graph_add_reverse",
]

lib_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libfusiongpu.so")

_c = ctypes
_vp, _i32, _i64, _u64, _f32, _f64, _sz = (_c.c_void_p, _c.c_int, _c.c_int64, _c.c_uint64, _c.c_float,
                                          _c.c_double, _c.c_size_t)

_SIGS = {
    "fgpu_last_error": (_c.c_char_p, []),
    "fgpu_abi_version": (_i32, []),
    "fgpu_index_create": (_i32, [_i32, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _c.POINTER(_vp)]),
    "fgpu_index_load": (_i32, [_c.c_char_p, _c.c_char_p, _i32, _i32, _c.POINTER(_vp)]),
    "fgpu_index_destroy": (None, [_vp]),
    "fgpu_index_get_info": (_i32, [_vp, _vp]),
    "fgpu_index_wrap": (_i32, [_i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _c.POINTER(_vp)]),
    "fgpu_index_faults": (_i32, [_vp, _vp, _c.POINTER(_c.c_ulonglong), _i32]),
    "fgpu_index_check": (_i32, [_vp, _vp]),
    "fgpu_debug_pq_sample": (_i32, [_i64, _i32, _vp]),
    "fgpu_stream_read_grid": (_i32, []),
    "fgpu_stream_read": (_i32, [_vp, _sz, _vp, _vp]),
    "fgpu_row_gather": (_i32, [_vp, _i64, _i32, _vp, _i64, _vp, _vp]),
    "fgpu_row_gather_lanes": (_i32, [_vp, _i64, _i32, _vp, _i64, _i32, _vp, _vp]),
    "fgpu_coarse_workspace_bytes": (_sz, [_i32, _i32]),
    "fgpu_coarse_search": (_i32, [_vp, _vp, _i32, _i32, _f32, _vp, _vp, _vp, _sz, _vp]),
    "fgpu_coarse_graph_workspace_bytes": (_sz, [_i32, _i32]),
    "fgpu_coarse_graph_build": (_i32, [_vp, _i32, _vp, _vp, _sz, _vp]),
    "fgpu_coarse_graph_search": (_i32, [_vp, _vp, _i32, _i32, _i32, _vp, _i32, _i32, _i32, _i32, _u64, _f32, _vp,
                                        _vp, _vp]),
    "fgpu_prune_probes": (_i32, [_vp, _vp, _i32, _i32, _f32, _vp]),
    "fgpu_probe_counts": (_i32, [_vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "fgpu_adc_search": (_i32, [_vp, _vp, _i32, _vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "fgpu_adc_search_stats": (_i32, [_vp, _vp, _i32, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp]),
    "fgpu_search_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "fgpu_search": (_i32, [_vp, _vp, _i32, _i32, _i32, _f32, _vp, _vp, _vp, _sz, _vp]),
    "fgpu_search_screen_stats": (_i32, [_vp, _i32, _i32, _vp, _sz, _vp, _c.POINTER(_c.c_longlong), _i32]),
    "fgpu_index_screen_ready": (_i32, [_vp]),
    "fgpu_index_set_option": (_i32, [_vp, _i32, _i32]),
    "fgpu_coarse_search_stats": (_i32, [_vp, _vp, _i32, _i32, _f32, _vp, _vp, _vp, _vp, _sz, _vp]),
    "fgpu_two_phase_search_precut": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp, _vp,
                                            _vp, _vp, _vp, _sz, _vp]),
    "fgpu_rerank_state": (_i32, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp,
                                 _vp, _vp, _i32, _vp]),
    "fgpu_graph_add_reverse": (_i32, [_vp, _i64, _i32, _i32, _vp, _i32]),
    "fgpu_search_stage_times": (_i32, [_vp, _c.POINTER(_c.c_float), _i32]),
    "fgpu_search_noalloc_max_bytes": (_sz, []),
    "fgpu_search_noalloc_max_rows": (_i32, [_i32, _i32]),
    "fgpu_search_noalloc": (_i32, [_vp, _vp, _i32, _i32, _i32, _f32, _vp, _vp, _vp]),
    "fgpu_two_phase_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "fgpu_two_phase_search": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp, _vp, _vp,
                                     _vp, _sz, _vp]),
    "fgpu_two_phase_search_stats": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp, _vp,
                                           _vp, _sz, _vp]),
    "fgpu_rerank": (_i32, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp, _vp]),
    "fgpu_rerank_spec": (_i32, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _vp,
                                _i32, _vp]),
    "fgpu_search_rerank_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "fgpu_search_rerank": (_i32, [_vp, _vp, _i32, _i32, _f32, _i32, _i32, _f32, _i32, _vp, _i64, _i32, _i32, _f32,
                                  _i32, _vp, _vp, _vp, _sz, _vp]),
    "fgpu_knn_exact_workspace_bytes": (_sz, [_i32, _i64]),
    "fgpu_knn_exact": (_i32, [_vp, _i32, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "fgpu_graph_search": (_i32, [_vp, _i32, _vp, _i64, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _u64, _vp, _vp, _vp,
                                 _vp, _vp]),
    "fgpu_l2_topk_workspace_bytes": (_sz, [_i64, _i32]),
    "fgpu_l2_topk": (_i32, [_vp, _i64, _vp, _i32, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "fgpu_kmeans_workspace_bytes": (_sz, [_i32, _i32]),
    "fgpu_kmeans_update": (_i32, [_vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "fgpu_fixed_shift": (_i32, [_f32, _i64]),
    "fgpu_tune_list_stats": (_i32, [_vp, _vp, _i32, _vp, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp,
                                    _vp]),
    "fgpu_tune_percentile_int": (_i32, [_vp, _i64, _f32]),
    "fgpu_tune_percentile": (_f32, [_vp, _i64, _f32]),
    "fgpu_tune_elbow": (_i32, [_vp, _i32, _i64, _c.POINTER(_f32)]),
    "fgpu_kmeans_fit": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _u64, _vp, _vp, _vp]),
    "fgpu_pq_train": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp, _i32, _i32, _vp, _vp]),
    "fgpu_pq_encode": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "fgpu_pq_encode_form": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp, _vp, _i32, _vp, _vp]),
    "fgpu_build_ivfpq": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _i32, _u64, _i32, _i32,
                                _vp, _vp, _vp, _vp, _vp, _vp]),
    "fgpu_build_ivfpq_sampled": (_i32, [_vp, _i64, _i32, _i32, _i32, _i64, _i32, _i32, _u64, _i32, _i32,
                                        _vp, _vp, _vp, _vp, _vp, _vp]),
    "fgpu_write_ivf_data": (_i32, [_c.c_char_p, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "fgpu_read_ivf_header": (_i32, [_c.c_char_p, _c.POINTER(_i64), _c.POINTER(_i32)]),
    "fgpu_read_ivf_data": (_i32, [_c.c_char_p, _i32, _i32, _vp, _vp, _vp, _vp]),
    "fgpu_write_fvecs": (_i32, [_c.c_char_p, _vp, _i64, _i32]),
    "fgpu_read_fvecs": (_i32, [_c.c_char_p, _i32, _c.POINTER(_i64), _vp]),
    "fgpu_read_ivecs": (_i32, [_c.c_char_p, _c.POINTER(_i32), _c.POINTER(_i64), _vp]),
    "fgpu_gen_gmm": (None, [_i64, _i32, _i32, _f64, _f64, _f64, _f64, _u64, _i32, _vp, _i32]),
}


class FgpuError(RuntimeError):
    """A libfusiongpu call returned a non-zero fgpu_status."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"fgpu status {status}: {msg}")
        self.status = status


def _load():
    if not os.path.exists(lib_path):
        raise ImportError(f"{lib_path} is not built; run __graft_entry__.build() (hipcc for gfx950)")
    # torch ships its own libamdhip64.so.7.  Importing torch first makes this
    # library bind to that already-loaded HIP runtime instead of loading a
    # second one (/opt/rocm) into the process: two runtimes cannot share the
    # device, and the second reports "no ROCm-capable device".
    import torch  # noqa: F401,PLC0415
    l = ctypes.CDLL(lib_path)
    for name, (res, args) in _SIGS.items():
        f = getattr(l, name)
        f.restype = res
        f.argtypes = args
    return l


lib = _load()


def _check(st: int):
    if st != 0:
        raise FgpuError(st, lib.fgpu_last_error().decode(errors="replace"))


def _np_ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_vp)


# --------------------------------------------------------------------------- torch plumbing
def _torch():
    import torch  # noqa: PLC0415 -- only needed for device buffers
    return torch


FAULT_ID = -2  # FGPU_FAULT_ID: every slot of a query a bounded-wait give-up may have touched


def _dev_ptr(t):
    assert t.is_cuda and t.is_contiguous(), "expected a contiguous device tensor"
    return _vp(t.data_ptr())


def _opt_ptr(t):
    return _dev_ptr(t) if t is not None else None


def _on(stream):
    """Context for one library call: with an explicit stream, that stream is
    torch's current stream while the call converts its inputs, allocates its
    workspace, temporaries and outputs and enqueues its kernels.  The caching
    allocator then ties every internal tensor to the stream the kernels run on,
    so memory freed when the call returns is only handed to later work on that
    same stream, never to other work while the kernels still read it."""
    if stream is None:
        return contextlib.nullcontext()
    return _torch().cuda.stream(stream)


def _stream():
    """hipStream_t of torch's current stream (the one _on made current)."""
    return _vp(_torch().cuda.current_stream().cuda_stream)


def _workspace(nbytes: int):
    torch = _torch()
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device="cuda")


def _ws_check(ws, name="workspace"):
    torch = _torch()
    if not (torch.is_tensor(ws) and ws.is_cuda and ws.is_contiguous()):
        raise ValueError(f"{name}: expected a contiguous device tensor")
    return ws.numel() * ws.element_size()


# Implicit conversions the host mirror performs (the C ABI reads exactly these
# element types): floating inputs become float32, integer ids int32.  An
# integer value must fit in int32, except 0xFFFFFFFF (the pruned-probe
# sentinel of a uint32 or int64 probe array), which becomes -1; any other
# value outside int32 raises ValueError instead of wrapping.
_FLOATS = ("float64", "float16", "bfloat16")
_INTS = ("int64", "int16", "int8", "uint8", "uint16", "uint32")
_INT32_MIN, _INT32_MAX, _PRUNED = -(1 << 31), (1 << 31) - 1, 0xFFFFFFFF


def _check_int32_range(a, name):
    torch = _torch()
    if a.numel() == 0 or str(a.dtype).replace("torch.", "") in ("int16", "int8", "uint8", "uint16"):
        return
    v = a.to(torch.int64) if a.dtype == torch.uint32 else a
    bad = ((v < _INT32_MIN) | (v > _INT32_MAX)) & (v != _PRUNED)
    if bool(bad.any()):
        first = int(v[bad].flatten()[0])
        raise ValueError(f"{name}: value {first} does not fit in int32 (the C ABI reads int32 ids)")


def _arg(a, dtype, name, shape=None):
    """`a` (numpy array or torch tensor) as a torch tensor of `dtype` where it
    lies, after checking its rank and the fixed entries of `shape` (None = any
    size).  Raises TypeError / ValueError before anything is copied."""
    torch = _torch()
    if isinstance(a, np.ndarray):
        a = torch.from_numpy(np.ascontiguousarray(a))
    elif not torch.is_tensor(a):
        raise TypeError(f"{name}: expected a numpy array or a torch tensor, got {type(a).__name__}")
    if a.dtype != dtype:
        src = str(a.dtype).replace("torch.", "")
        ok = (dtype == torch.float32 and src in _FLOATS) or (dtype == torch.int32 and src in _INTS)
        if not ok:
            raise TypeError(f"{name}: dtype {src} cannot be read as {str(dtype).replace('torch.', '')}")
        if dtype == torch.int32:
            _check_int32_range(a, name)
    if shape is not None:
        if a.dim() != len(shape):
            raise ValueError(f"{name}: expected {len(shape)} dimensions, got shape {tuple(a.shape)}")
        for i, want in enumerate(shape):
            if want is not None and a.shape[i] != want:
                raise ValueError(f"{name}: dimension {i} is {a.shape[i]}, expected {want} "
                                 f"(shape {tuple(a.shape)})")
    return a.to(dtype) if a.dtype != dtype else a


def _dev(a, dtype, name, shape=None):
    """_arg, then a contiguous device tensor (copied to the device if needed)."""
    a = _arg(a, dtype, name, shape)
    if not a.is_cuda:
        a = a.to("cuda")
    return a.contiguous()


def _out(t, dtype, shape, name):
    """Check a caller-supplied output tensor (dtype, exact shape, contiguous device memory)."""
    torch = _torch()
    if not torch.is_tensor(t):
        raise TypeError(f"{name}: expected a torch tensor")
    if t.dtype != dtype or tuple(t.shape) != tuple(shape) or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous device tensor {str(dtype).replace('torch.', '')}"
                         f"{list(shape)}, got {t.dtype} {list(t.shape)} on {t.device}")
    return t


def _outs(out, nq, k, name="out"):
    """(ids int32 [nq][k], dists float32 [nq][k]): the caller's, checked, or new."""
    torch = _torch()
    if out is None:
        return (torch.empty((nq, k), dtype=torch.int32, device="cuda"),
                torch.empty((nq, k), dtype=torch.float32, device="cuda"))
    ids, d = out
    return _out(ids, torch.int32, (nq, k), name + "[0]"), _out(d, torch.float32, (nq, k), name + "[1]")


# --------------------------------------------------------------------------- synthetic data
def gen_gmm(n: int, dim: int, ncomp: int, seed: int, set: int = 0, lo: float = -1.0, hi: float = 1.0,
            sig_lo: float = 0.1, sig_hi: float | None = None, nthreads: int = 0) -> np.ndarray:
    """Seeded Gaussian-mixture vectors [n][dim] float32 (set 0 = base, 1 = queries)."""
    out = np.empty((n, dim), np.float32)
    lib.fgpu_gen_gmm(n, dim, ncomp, lo, hi, sig_lo, sig_lo if sig_hi is None else sig_hi, seed, set,
                     _np_ptr(out), nthreads)
    return out


# --------------------------------------------------------------------------- files
def write_ivf_data(path, offsets, ids, codes, centroids):
    offsets = np.ascontiguousarray(offsets, np.int32)
    ids = np.ascontiguousarray(ids, np.int32)
    codes = np.ascontiguousarray(codes, np.uint8)
    centroids = np.ascontiguousarray(centroids, np.float32)
    _check(lib.fgpu_write_ivf_data(str(path).encode(), ids.shape[0], offsets.shape[0] - 1, codes.shape[1],
                                   centroids.shape[1], _np_ptr(offsets), _np_ptr(ids), _np_ptr(codes),
                                   _np_ptr(centroids)))


def read_ivf_data(path, pq_m: int, dim: int):
    total, nlist = _i64(), _i32()
    _check(lib.fgpu_read_ivf_header(str(path).encode(), _c.byref(total), _c.byref(nlist)))
    offs = np.empty(nlist.value + 1, np.int32)
    ids = np.empty(total.value, np.int32)
    codes = np.empty((total.value, pq_m), np.uint8)
    cent = np.empty((nlist.value, dim), np.float32)
    _check(lib.fgpu_read_ivf_data(str(path).encode(), pq_m, dim, _np_ptr(offs), _np_ptr(ids), _np_ptr(codes),
                                  _np_ptr(cent)))
    return offs, ids, codes, cent


def write_fvecs(path, v):
    v = np.ascontiguousarray(v, np.float32)
    _check(lib.fgpu_write_fvecs(str(path).encode(), _np_ptr(v), v.shape[0], v.shape[1]))


def read_fvecs(path, dim: int) -> np.ndarray:
    n = _i64()
    _check(lib.fgpu_read_fvecs(str(path).encode(), dim, _c.byref(n), None))
    out = np.empty((n.value, dim), np.float32)
    _check(lib.fgpu_read_fvecs(str(path).encode(), dim, _c.byref(n), _np_ptr(out)))
    return out


def read_ivecs(path) -> np.ndarray:
    d, n = _i32(), _i64()
    _check(lib.fgpu_read_ivecs(str(path).encode(), _c.byref(d), _c.byref(n), None))
    out = np.empty((n.value, d.value), np.int32)
    _check(lib.fgpu_read_ivecs(str(path).encode(), _c.byref(d), _c.byref(n), _np_ptr(out)))
    return out


def debug_pq_sample(n: int, sample_size: int) -> np.ndarray:
    """Test hook (fgpu_debug_pq_sample, host only): fgpu_pq_train's sample rows."""
    out = np.empty(max(0, min(int(sample_size), int(n))), dtype=np.int32)
    got = lib.fgpu_debug_pq_sample(int(n), int(sample_size), out.ctypes.data)
    if got < 0:
        raise ValueError("debug_pq_sample: bad argument")
    return out[:got]


def stream_read(data, stream=None):
    """Stream a contiguous device tensor through 16-byte loads (fgpu_stream_read), for a measured read rate."""
    torch = _torch()
    with _on(stream):
        if not (torch.is_tensor(data) and data.is_cuda and data.is_contiguous()):
            raise ValueError("stream_read: expected a contiguous device tensor")
        sink = torch.empty(lib.fgpu_stream_read_grid(), dtype=torch.int64, device="cuda")
        _check(lib.fgpu_stream_read(_dev_ptr(data), data.numel() * data.element_size(), _dev_ptr(sink), _stream()))


def row_gather(rows, idx, lanes_per_row=8, stream=None):
    """Read whole rows rows[idx[i]] (384- or 512-byte rows of a contiguous 2-D device tensor), eight lanes a row
    (the library's pattern) or one (fgpu_row_gather_lanes), for a measured random-row read rate."""
    torch = _torch()
    with _on(stream):
        if not (torch.is_tensor(rows) and rows.is_cuda and rows.is_contiguous() and rows.dim() == 2):
            raise ValueError("row_gather: expected a contiguous 2-D device tensor")
        ix = _dev(idx, torch.int32, "idx", (None,))
        sink = torch.empty(lib.fgpu_stream_read_grid(), dtype=torch.int64, device="cuda")
        _check(lib.fgpu_row_gather_lanes(_dev_ptr(rows), rows.shape[0], rows.shape[1] * rows.element_size(),
                                         _dev_ptr(ix), ix.shape[0], int(lanes_per_row), _dev_ptr(sink), _stream()))


# --------------------------------------------------------------------------- index + search
class _Info(ctypes.Structure):
    _fields_ = [("dim", _i32), ("pq_m", _i32), ("pq_k", _i32), ("nlist", _i32), ("total", _i64),
                ("d_pq_codebook", _vp), ("d_cluster_offsets", _vp), ("d_all_pq_codes", _vp),
                ("d_all_vector_ids", _vp), ("d_centroids", _vp), ("max_list_len", _i32)]


class Index:
    """Device-resident IVF-PQ index (the reference's IVFIndexGPU, defs.h:51-58)."""

    def __init__(self, handle):
        self._h = _vp(handle)
        info = _Info()
        _check(lib.fgpu_index_get_info(self._h, _c.byref(info)))
        self.dim, self.pq_m, self.nlist, self.total = info.dim, info.pq_m, info.nlist, info.total
        self.max_list_len = info.max_list_len
        self.info = info

    @classmethod
    def from_arrays(cls, dim, pq_m, offsets, ids, codes, centroids, codebook) -> "Index":
        offsets = np.ascontiguousarray(offsets, np.int32)
        ids = np.ascontiguousarray(ids, np.int32)
        codes = np.ascontiguousarray(codes, np.uint8)
        centroids = np.ascontiguousarray(centroids, np.float32)
        codebook = np.ascontiguousarray(codebook, np.float32)
        nlist, total = offsets.shape[0] - 1, ids.shape[0]
        if codes.shape != (total, pq_m) or centroids.shape != (nlist, dim) or codebook.size != pq_m * 256 * (
                dim // max(pq_m, 1)):
            raise ValueError(f"from_arrays: inconsistent shapes: ids {ids.shape}, codes {codes.shape}, "
                             f"centroids {centroids.shape}, codebook {codebook.shape} for dim {dim}, pq_m {pq_m}")
        h = _vp()
        _check(lib.fgpu_index_create(dim, pq_m, nlist, total, _np_ptr(offsets), _np_ptr(ids), _np_ptr(codes),
                                     _np_ptr(centroids), _np_ptr(codebook), _c.byref(h)))
        return cls(h.value)

    @classmethod
    def wrap(cls, dim, pq_m, offsets, ids, codes, centroids, codebook, stream=None) -> "Index":
        """An index over device tensors the caller keeps (fgpu_index_wrap): no copy of the A1 arrays.  The
        tensors are held by the returned object, so they outlive its handle."""
        torch = _torch()
        with _on(stream):
            offsets = _dev(offsets, torch.int32, "offsets", (None,))
            nlist = offsets.shape[0] - 1
            ids = _dev(ids, torch.int32, "ids", (None,))
            codes = _dev(codes, torch.uint8, "codes", (ids.shape[0], pq_m))
            centroids = _dev(centroids, torch.float32, "centroids", (nlist, dim))
            codebook = _dev(codebook, torch.float32, "codebook", (pq_m, 256, dim // max(pq_m, 1)))
            h = _vp()
            _check(lib.fgpu_index_wrap(dim, pq_m, nlist, _dev_ptr(offsets), _dev_ptr(ids), _dev_ptr(codes),
                                       _dev_ptr(centroids), _dev_ptr(codebook), _stream(), _c.byref(h)))
        ix = cls(h.value)
        ix._arrays = (offsets, ids, codes, centroids, codebook)
        return ix

    @classmethod
    def load(cls, ivf_data_path, codebook_path, dim: int, pq_m: int) -> "Index":
        h = _vp()
        _check(lib.fgpu_index_load(str(ivf_data_path).encode(), str(codebook_path).encode(), dim, pq_m,
                                   _c.byref(h)))
        return cls(h.value)

    def close(self):
        if self._h:
            lib.fgpu_index_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- bounded-wait give-ups of the scan kernel
    def faults(self, reset: bool = False, stream=None) -> int:
        """Give-ups of the scan kernel's bounded waits on this index (fgpu_index_faults; 0 in a correct run).
        Waits for the stream."""
        v = _c.c_ulonglong()
        with _on(stream):
            _check(lib.fgpu_index_faults(self._h, _stream(), _c.byref(v), int(bool(reset))))
        return int(v.value)

    def check(self, stream=None):
        """Raise FgpuError (FGPU_ERR_WAIT) if any bounded wait of the scan kernel gave up (fgpu_index_check)."""
        with _on(stream):
            _check(lib.fgpu_index_check(self._h, _stream()))

    # -- argument helpers
    def _queries(self, queries):
        return _dev(queries, _torch().float32, "queries", (None, self.dim))

    def _probes(self, probe_ids, nq=None):
        p = _dev(probe_ids, _torch().int32, "probe_ids", (nq, None))
        if p.shape[1] < 1:
            raise ValueError("probe_ids: need at least one probe per query")
        return p

    # -- search
    def coarse_workspace_bytes(self, nq: int) -> int:
        return lib.fgpu_coarse_workspace_bytes(nq, self.nlist)

    def coarse_search(self, queries, nprobe: int, prune_ratio: float = 100.0, workspace=None, out=None,
                      stream=None):
        """Exact top-nprobe lists: (probe_ids uint32-as-int32 [nq][nprobe], dists [nq][nprobe])."""
        with _on(stream):
            q = self._queries(queries)
            nq = q.shape[0]
            ws = workspace if workspace is not None else _workspace(self.coarse_workspace_bytes(nq))
            ids, d = _outs(out, nq, nprobe)
            _check(lib.fgpu_coarse_search(self._h, _dev_ptr(q), nq, nprobe, prune_ratio, _dev_ptr(ids), _dev_ptr(d),
                                          _dev_ptr(ws), _ws_check(ws), _stream()))
        return ids, d

    def coarse_search_stats(self, queries, nprobe: int, prune_ratio: float = 100.0, stream=None):
        """coarse_search plus counters (fgpu_coarse_search_stats): (probe_ids, dists, {"rescored": centroids
        re-scored exactly, summed over the queries, "full_rows": queries that re-scored every centroid})."""
        torch = _torch()
        with _on(stream):
            q = self._queries(queries)
            nq = q.shape[0]
            ws = _workspace(self.coarse_workspace_bytes(nq))
            ids, d = _outs(None, nq, nprobe)
            st = torch.zeros(2, dtype=torch.int64, device="cuda")
            _check(lib.fgpu_coarse_search_stats(self._h, _dev_ptr(q), nq, nprobe, prune_ratio, _dev_ptr(ids),
                                                _dev_ptr(d), _dev_ptr(st), _dev_ptr(ws), _ws_check(ws), _stream()))
            v = st.cpu().tolist()
        return ids, d, {"rescored": v[0], "full_rows": v[1]}

    def coarse_graph_build(self, degree: int = 8, stream=None):
        """Exact kNN graph of the centroids, self excluded (fgpu_coarse_graph_build): int32 [nlist][degree]."""
        torch = _torch()
        with _on(stream):
            g = torch.empty((self.nlist, degree), dtype=torch.int32, device="cuda")
            ws = _workspace(lib.fgpu_coarse_graph_workspace_bytes(self.nlist, degree))
            _check(lib.fgpu_coarse_graph_build(self._h, degree, _dev_ptr(g), _dev_ptr(ws), _ws_check(ws), _stream()))
        return g

    def coarse_graph_search(self, queries, nprobe: int, graph, itopk: int = 32, width: int = 4, max_iter: int = 200,
                            seed: int = 1, prune_ratio: float = 100.0, first_query: int = 0, out=None,
                            stream=None):
        """Top-nprobe lists by the graph walk over the centroids (fgpu_coarse_graph_search): (probe_ids
        uint32-as-int32 [nq][nprobe], dists [nq][nprobe])."""
        torch = _torch()
        with _on(stream):
            q = self._queries(queries)
            g = _dev(graph, torch.int32, "graph", (self.nlist, None))
            nq = q.shape[0]
            ids, d = _outs(out, nq, nprobe)
            _check(lib.fgpu_coarse_graph_search(self._h, _dev_ptr(q), nq, first_query, nprobe, _dev_ptr(g),
                                                g.shape[1], itopk, width, max_iter, seed, prune_ratio, _dev_ptr(ids),
                                                _dev_ptr(d), _stream()))
        return ids, d

    def adc_search(self, queries, probe_ids, k: int, out=None, stream=None, probe_dists=None):
        """LUT + ADC scan + top-k over the probed lists: (ids int32 [nq][k], dists float32 [nq][k]).
        probe_dists: coarse_search's distances for these probes (optional; the list bounds use them)."""
        torch = _torch()
        with _on(stream):
            q = self._queries(queries)
            nq = q.shape[0]
            p = self._probes(probe_ids, nq)
            nprobe = p.shape[1]
            pd = _dev(probe_dists, torch.float32, "probe_dists", (nq, nprobe)) if probe_dists is not None else None
            ids, d = _outs(out, nq, k)
            _check(lib.fgpu_adc_search(self._h, _dev_ptr(q), nq, _dev_ptr(p), _opt_ptr(pd), nprobe, k, _dev_ptr(ids),
                                       _dev_ptr(d), _stream()))
        return ids, d

    def adc_search_stats(self, queries, probe_ids, k: int, out=None, stream=None, probe_dists=None):
        """adc_search plus counters: (ids, dists, {"vectors_loaded", "luts_built", "lists_skipped", clocks})."""
        torch = _torch()
        with _on(stream):
            q = self._queries(queries)
            nq = q.shape[0]
            p = self._probes(probe_ids, nq)
            nprobe = p.shape[1]
            pd = _dev(probe_dists, torch.float32, "probe_dists", (nq, nprobe)) if probe_dists is not None else None
            ids, d = _outs(out, nq, k)
            st = torch.zeros(8, dtype=torch.int64, device="cuda")
            _check(lib.fgpu_adc_search_stats(self._h, _dev_ptr(q), nq, _dev_ptr(p), _opt_ptr(pd), nprobe, k,
                                             _dev_ptr(ids), _dev_ptr(d), _dev_ptr(st), _stream()))
            v = st.cpu().tolist()
        return ids, d, {"vectors_loaded": v[0], "luts_built": v[1], "lists_skipped": v[2], "clk_setup": v[3],
                        "clk_builder": v[4], "clk_scanner": v[5], "clk_total": v[6]}

    def two_phase_search(self, queries, probe_ids, p1_lists: int, limit_k: int, threshold_coeff: float,
                         rerank_m: int, want_cutoffs: bool = False, workspace=None, stream=None,
                         want_pre_cut: bool = False):
        """run_gpu_batch_logic after the coarse step: (top_ids [nq][rerank_m], top_dists, top_counts [nq],
        cutoffs [nq][p1] or None, thresholds [nq] or None) and, with want_pre_cut, each query's candidate count
        before the rerank_m cut (fgpu_two_phase_search_precut; the reference's d_atomic)."""
        torch = _torch()
        with _on(stream):
            q = self._queries(queries)
            nq = q.shape[0]
            p = self._probes(probe_ids, nq)
            nprobe = p.shape[1]
            p1 = max(0, min(nprobe, p1_lists))
            ws = workspace if workspace is not None else _workspace(
                lib.fgpu_two_phase_workspace_bytes(nq, nprobe, p1_lists, limit_k, rerank_m))
            tid = torch.empty((nq, rerank_m), dtype=torch.int32, device="cuda")
            td = torch.empty((nq, rerank_m), dtype=torch.float32, device="cuda")
            tc = torch.empty(nq, dtype=torch.int32, device="cuda")
            cut = torch.empty((nq, max(p1, 1)), dtype=torch.float32, device="cuda") if want_cutoffs else None
            thr = torch.empty(nq, dtype=torch.float32, device="cuda") if want_cutoffs else None
            if want_pre_cut:
                pre = torch.empty(nq, dtype=torch.int32, device="cuda")
                _check(lib.fgpu_two_phase_search_precut(self._h, _dev_ptr(q), nq, _dev_ptr(p), nprobe, p1_lists,
                                                        limit_k, threshold_coeff, rerank_m, _dev_ptr(tid),
                                                        _dev_ptr(td), _dev_ptr(tc), _opt_ptr(cut), _opt_ptr(thr),
                                                        _dev_ptr(pre), _dev_ptr(ws), _ws_check(ws), _stream()))
                return tid, td, tc, (cut[:, :p1] if want_cutoffs else None), thr, pre
            _check(lib.fgpu_two_phase_search(self._h, _dev_ptr(q), nq, _dev_ptr(p), nprobe, p1_lists, limit_k,
                                             threshold_coeff, rerank_m, _dev_ptr(tid), _dev_ptr(td), _dev_ptr(tc),
                                             _opt_ptr(cut), _opt_ptr(thr), _dev_ptr(ws), _ws_check(ws), _stream()))
        return tid, td, tc, (cut[:, :p1] if want_cutoffs else None), thr

    def two_phase_stats(self, queries, probe_ids, p1_lists: int, limit_k: int, threshold_coeff: float, rerank_m: int,
                        workspace=None, stream=None):
        """two_phase_search plus counters: (top_ids, top_dists, top_counts, {counter: value})."""
        torch = _torch()
        with _on(stream):
            q = self._queries(queries)
            nq = q.shape[0]
            p = self._probes(probe_ids, nq)
            nprobe = p.shape[1]
            ws = workspace if workspace is not None else _workspace(
                lib.fgpu_two_phase_workspace_bytes(nq, nprobe, p1_lists, limit_k, rerank_m))
            tid = torch.empty((nq, rerank_m), dtype=torch.int32, device="cuda")
            td = torch.empty((nq, rerank_m), dtype=torch.float32, device="cuda")
            tc = torch.empty(nq, dtype=torch.int32, device="cuda")
            st = torch.zeros(20, dtype=torch.int64, device="cuda")
            _check(lib.fgpu_two_phase_search_stats(self._h, _dev_ptr(q), nq, _dev_ptr(p), nprobe, p1_lists, limit_k,
                                                   threshold_coeff, rerank_m, _dev_ptr(tid), _dev_ptr(td),
                                                   _dev_ptr(tc), _dev_ptr(st), _dev_ptr(ws), _ws_check(ws),
                                                   _stream()))
            v = st.cpu().tolist()
        return tid, td, tc, {"vectors_loaded": v[0], "luts_built": v[1], "lists_skipped": v[2],
                             "phase2_appended": v[3], "clk_setup": v[4], "clk_phase1": v[5], "clk_phase2": v[6],
                             "clk_final": v[7], "clk_p1_build": v[8], "clk_p1_scan": v[9], "clk_p1_merge": v[10],
                             "screen_virtual_queries": v[11], "screen_candidates": v[12], "screen_to_lut": v[13],
                             "screen_no_threshold": v[14], "screen_over_cap": v[15],
                             "screen_vector_pairs_round1": v[16], "screen_vector_pairs_round2": v[17],
                             "screen_tiles_round1": v[18], "screen_tiles_round2": v[19]}

    def search_rerank_workspace_bytes(self, nq: int, nprobe: int, p1_lists: int, limit_k: int, rerank_m: int) -> int:
        return lib.fgpu_search_rerank_workspace_bytes(nq, self.nlist, nprobe, p1_lists, limit_k, rerank_m)

    def search_rerank(self, queries, base, nprobe: int, k: int, p1_lists: int = 12, limit_k: int = 50,
                      threshold_coeff: float = 1.0, rerank_m: int = 1000, mini_batch: int = 128, eps: float = 0.1,
                      beta: int = 2, prune_ratio: float = 100.0, workspace=None, out=None, stream=None):
        """coarse + two-phase scan + exact rerank (SearchPipeline's per-batch path): (ids, dists) [nq][k]."""
        torch = _torch()
        with _on(stream):
            q = self._queries(queries)
            b = _dev(base, torch.float32, "base", (None, self.dim))
            nq = q.shape[0]
            ws = workspace if workspace is not None else _workspace(
                self.search_rerank_workspace_bytes(nq, nprobe, p1_lists, limit_k, rerank_m))
            ids, d = _outs(out, nq, k)
            _check(lib.fgpu_search_rerank(self._h, _dev_ptr(q), nq, nprobe, prune_ratio, p1_lists, limit_k,
                                          threshold_coeff, rerank_m, _dev_ptr(b), b.shape[0], k, mini_batch, eps, beta,
                                          _dev_ptr(ids), _dev_ptr(d), _dev_ptr(ws), _ws_check(ws), _stream()))
        return ids, d

    def search_workspace_bytes(self, nq: int, nprobe: int) -> int:
        return lib.fgpu_search_workspace_bytes(nq, self.nlist, nprobe)

    def search(self, queries, nprobe: int, k: int, prune_ratio: float = 100.0, workspace=None, out=None,
               stream=None):
        """coarse + scan + top-k in one call (fgpu_search; the MFMA screen with an exact rescore where it
        applies, the LUT kernels otherwise): (ids int32 [nq][k], dists float32 [nq][k])."""
        with _on(stream):
            q = self._queries(queries)
            nq = q.shape[0]
            ws = workspace if workspace is not None else _workspace(self.search_workspace_bytes(nq, nprobe))
            ids, d = _outs(out, nq, k)
            _check(lib.fgpu_search(self._h, _dev_ptr(q), nq, nprobe, k, prune_ratio, _dev_ptr(ids), _dev_ptr(d),
                                   _dev_ptr(ws), _ws_check(ws), _stream()))
        return ids, d

    OPT_LIST_SKIP, OPT_SPIN_LIMIT, OPT_SCREEN, OPT_SCREEN_CLOCKS, OPT_TWO_PHASE_SPLIT, OPT_STAGE_EVENTS = \
        1, 2, 3, 4, 5, 6
    OPT_TWO_PHASE_SCREEN = 7
    STAGES = ("coarse", "screen_pairs1", "screen_round1", "screen_pairs2", "screen_round2", "rescore", "lut_kernel")

    def set_option(self, option: int, value: int):
        """Per-index option (fgpu_index_set_option): OPT_LIST_SKIP (0 = the LUT scan reads every probed list),
        OPT_SPIN_LIMIT (polls before a flow-kernel wait gives up, 0 = automatic), OPT_SCREEN (0 = fgpu_search
        runs the LUT kernels), OPT_SCREEN_CLOCKS (1 = the screen records shader clocks),
        OPT_TWO_PHASE_SPLIT (phase-1 workgroups a query: 0 automatic, 1 never, s >= 2), OPT_STAGE_EVENTS
        (1 = search records HIP events between its stages, read by search_stage_times), OPT_TWO_PHASE_SCREEN
        (two-phase phase 1 through the MFMA screen: 0 automatic for batches >= 1024, 1 never, 2 always).
        Results never depend on them; they change only this index's later calls."""
        _check(lib.fgpu_index_set_option(self._h, int(option), int(value)))

    @property
    def screen_ready(self) -> bool:
        """Whether the index carries the MFMA screen's arrays (fgpu_index_screen_ready)."""
        return bool(lib.fgpu_index_screen_ready(self._h))

    def search_screen_stats(self, nq: int, nprobe: int, workspace, stream=None) -> dict:
        """Counters of the last search() on `workspace` that took the MFMA screen (fgpu_search_screen_stats;
        waits for the stream)."""
        st = (_c.c_longlong * 20)()
        with _on(stream):
            _check(lib.fgpu_search_screen_stats(self._h, nq, nprobe, _dev_ptr(workspace), _ws_check(workspace),
                                                _stream(), st, 20))
        keys = ("pairs_round1", "lists_round2", "pairs_round2", "candidates", "max_candidates",
                "queries_to_lut_kernel", "queries_with_threshold", "_",
                "clk1_pre", "clk1_setup", "clk1_tiles", "clk1_post", "clk2_pre", "clk2_setup", "clk2_tiles",
                "clk2_post", "vector_pairs_round1", "vector_pairs_round2", "tiles_round1", "tiles_round2")
        return {kk: int(st[i]) for i, kk in enumerate(keys)}

    def search_stage_times(self) -> dict:
        """Milliseconds of the last search()'s stages, from the events it recorded on its stream with
        OPT_STAGE_EVENTS on (fgpu_search_stage_times; waits for them): keys Index.STAGES."""
        ms = (_c.c_float * len(self.STAGES))()
        _check(lib.fgpu_search_stage_times(self._h, ms, len(self.STAGES)))
        return {kk: float(ms[i]) for i, kk in enumerate(self.STAGES)}

    TP_STAGES = ("virtual_queries", "screen_pairs1", "screen_round1", "screen_pairs2", "screen_round2", "rescore",
                 "lut_collect_phase2_final")

    def two_phase_stage_times(self) -> dict:
        """Milliseconds of the stages of the last two_phase_search() whose phase 1 ran through the screen (the last
        virtual-query chunk), from the events it recorded with OPT_STAGE_EVENTS on: keys Index.TP_STAGES."""
        ms = (_c.c_float * len(self.TP_STAGES))()
        _check(lib.fgpu_search_stage_times(self._h, ms, len(self.TP_STAGES)))
        return {kk: float(ms[i]) for i, kk in enumerate(self.TP_STAGES)}

    def search_noalloc(self, queries, nprobe: int, k: int, prune_ratio: float = 100.0, out=None, stream=None):
        """fgpu_search without a workspace (fgpu_search_noalloc): its scratch is the library's fixed per-GPU
        device array, so the call itself allocates nothing; with out= and device queries of the right dtype
        neither does this method.  Calls overlapping on one GPU race on that array."""
        with _on(stream):
            q = self._queries(queries)
            nq = q.shape[0]
            ids, d = _outs(out, nq, k)
            _check(lib.fgpu_search_noalloc(self._h, _dev_ptr(q), nq, nprobe, k, prune_ratio, _dev_ptr(ids),
                                           _dev_ptr(d), _stream()))
        return ids, d

    def tune_list_stats(self, queries, pair_query, pair_list, pair_target=None, pair_kth=None, base=None,
                        stream=None):
        """The tuner's per-(query, list) statistics (fgpu_tune_list_stats): (target_pq, target_exact, pq_rank,
        exact_rank, kth_pq) as device tensors; the first four are None without pair_target, the last without
        pair_kth."""
        torch = _torch()
        with _on(stream):
            q = self._queries(queries)
            pq = _dev(pair_query, torch.int32, "pair_query", (None,))
            n = pq.shape[0]
            pl = _dev(pair_list, torch.int32, "pair_list", (n,))
            pt = _dev(pair_target, torch.int32, "pair_target", (n,)) if pair_target is not None else None
            pk = _dev(pair_kth, torch.int32, "pair_kth", (n,)) if pair_kth is not None else None
            b = _dev(base, torch.float32, "base", (None, self.dim)) if base is not None else None
            f = lambda: torch.empty(n, dtype=torch.float32, device="cuda")  # noqa: E731
            i = lambda: torch.empty(n, dtype=torch.int32, device="cuda")  # noqa: E731
            tp, te, pr, er = (f(), f(), i(), i()) if pt is not None else (None, None, None, None)
            kp = f() if pk is not None else None
            _check(lib.fgpu_tune_list_stats(self._h, _dev_ptr(q), q.shape[0], _opt_ptr(b),
                                            b.shape[0] if b is not None else 0, _dev_ptr(pq), _dev_ptr(pl),
                                            _opt_ptr(pt), _opt_ptr(pk), n,
                                            *(_opt_ptr(t) for t in (tp, te, pr, er, kp)), _stream()))
        return tp, te, pr, er, kp


def prune_probes(probe_ids, probe_dists, prune_ratio: float, stream=None):
    """The reference's prune rule in place on a device int32 probe tensor (fgpu_prune_probes): a probe farther
    than its query's first distance * prune_ratio becomes 0xFFFFFFFF (-1 as int32)."""
    torch = _torch()
    with _on(stream):
        nq, nprobe = probe_ids.shape
        _out(probe_ids, torch.int32, (nq, nprobe), "probe_ids")
        d = _dev(probe_dists, torch.float32, "probe_dists", (nq, nprobe))
        _check(lib.fgpu_prune_probes(_dev_ptr(probe_ids), _dev_ptr(d), nq, nprobe, prune_ratio, _stream()))
    return probe_ids


def probe_counts(index: Index, probe_ids, stream=None):
    torch = _torch()
    with _on(stream):
        p = index._probes(probe_ids)
        nq, nprobe = p.shape
        counts = torch.empty(nq, dtype=torch.int32, device="cuda")
        offs = torch.empty(nq + 1, dtype=torch.int32, device="cuda")
        _check(lib.fgpu_probe_counts(index._h, _dev_ptr(p), nq, nprobe, _dev_ptr(counts), _dev_ptr(offs), _stream()))
    return counts, offs


def rerank(queries, base, top_ids, top_counts, k: int, mini_batch: int = 128, eps: float = 0.1, beta: int = 2,
           stream=None, spec: int = 0, want_state: bool = False):
    """run_gpu_rerank: exact L2 over the ADC-ordered candidates with the early stop: (ids, dists, visited) and,
    with want_state, the reference's stab[] (int32) and fin[] (uint8) as the walk leaves them
    (fgpu_rerank_state).  spec: mini-batches computed at once (0 automatic, 1, or 4); results do not depend
    on it."""
    torch = _torch()
    with _on(stream):
        q = _dev(queries, torch.float32, "queries", (None, None))
        nq, dim = q.shape
        b = _dev(base, torch.float32, "base", (None, dim))
        t = _dev(top_ids, torch.int32, "top_ids", (nq, None))
        c = _dev(top_counts, torch.int32, "top_counts", (nq,))
        rm = t.shape[1]
        ids = torch.empty((nq, k), dtype=torch.int32, device="cuda")
        d = torch.empty((nq, k), dtype=torch.float32, device="cuda")
        vis = torch.empty(nq, dtype=torch.int32, device="cuda")
        stab = torch.empty(nq, dtype=torch.int32, device="cuda") if want_state else None
        fin = torch.empty(nq, dtype=torch.uint8, device="cuda") if want_state else None
        _check(lib.fgpu_rerank_state(_dev_ptr(q), nq, dim, _dev_ptr(b), b.shape[0], _dev_ptr(t), _dev_ptr(c), rm,
                                     k, mini_batch, eps, beta, _dev_ptr(ids), _dev_ptr(d), _dev_ptr(vis),
                                     _opt_ptr(stab), _opt_ptr(fin), int(spec), _stream()))
    if want_state:
        return ids, d, vis, stab, fin
    return ids, d, vis


# --------------------------------------------------------------------------- exact selection + build
def l2_topk(x, c, p: int, stream=None):
    """p nearest rows of c for each row of x by exact device-form L2: (ids, dists)."""
    torch = _torch()
    with _on(stream):
        x = _dev(x, torch.float32, "x", (None, None))
        n, dim = x.shape
        c = _dev(c, torch.float32, "c", (None, dim))
        nc = c.shape[0]
        ws = _workspace(lib.fgpu_l2_topk_workspace_bytes(n, nc))
        ids = torch.empty((n, p), dtype=torch.int32, device="cuda")
        d = torch.empty((n, p), dtype=torch.float32, device="cuda")
        _check(lib.fgpu_l2_topk(_dev_ptr(x), n, _dev_ptr(c), nc, dim, p, _dev_ptr(ids), _dev_ptr(d), _dev_ptr(ws),
                                _ws_check(ws), _stream()))
    return ids, d


def tune_percentile(values, pct: float):
    """compute_percentile(_int) of the tuner (host): sorted[floor(n * pct)], clamped; 0 when empty."""
    v = np.ascontiguousarray(values)
    if v.dtype.kind in "iu":
        v = np.ascontiguousarray(v, np.int32)
        return int(lib.fgpu_tune_percentile_int(_np_ptr(v) if v.size else None, v.size, pct))
    v = np.ascontiguousarray(v, np.float32)
    return float(lib.fgpu_tune_percentile(_np_ptr(v) if v.size else None, v.size, pct))


def tune_elbow(hits_per_rank, total_hits: int):
    """find_elbow_point of the tuner (host): (recommended phase-1 list count, coverage there)."""
    h = np.ascontiguousarray(hits_per_rank, np.int32)
    cov = _c.c_float()
    e = lib.fgpu_tune_elbow(_np_ptr(h) if h.size else None, h.size, int(total_hits), _c.byref(cov))
    return int(e), float(cov.value)


def knn_exact(queries, base, k: int, workspace=None, stream=None):
    """Exact kNN ground truth (brute_force_search_kernel): (ids int32 [nq][k], dists float32 [nq][k])."""
    torch = _torch()
    with _on(stream):
        q = _dev(queries, torch.float32, "queries", (None, None))
        nq, dim = q.shape
        b = _dev(base, torch.float32, "base", (None, dim))
        n = b.shape[0]
        ws = workspace if workspace is not None else _workspace(lib.fgpu_knn_exact_workspace_bytes(nq, n))
        ids = torch.empty((nq, k), dtype=torch.int32, device="cuda")
        d = torch.empty((nq, k), dtype=torch.float32, device="cuda")
        _check(lib.fgpu_knn_exact(_dev_ptr(q), nq, _dev_ptr(b), n, dim, k, _dev_ptr(ids), _dev_ptr(d), _dev_ptr(ws),
                                  _ws_check(ws), _stream()))
    return ids, d


def graph_add_reverse(fwd, degree: int, nthreads: int = 0) -> np.ndarray:
    """CAGRA's reverse-edge step (fgpu_graph_add_reverse) on host arrays: fwd int32 [n][width], each row's
    forward candidates nearest first; returns int32 [n][degree]."""
    fwd = np.ascontiguousarray(fwd, np.int32)
    n, width = fwd.shape
    out = np.empty((n, degree), np.int32)
    _check(lib.fgpu_graph_add_reverse(_np_ptr(fwd), n, width, degree, _np_ptr(out), nthreads))
    return out


def graph_search(queries, base, graph, k: int, itopk: int = 64, width: int = 4, max_iter: int = 64, seed: int = 1,
                 want_evals: bool = False, out=None, stream=None):
    """Graph search over a fixed-degree adjacency (the CAGRA role): (ids [nq][k], dists [nq][k], steps [nq])
    plus, with want_evals, the exact distances computed per query."""
    torch = _torch()
    with _on(stream):
        q = _dev(queries, torch.float32, "queries", (None, None))
        nq, dim = q.shape
        b = _dev(base, torch.float32, "base", (None, dim))
        g = _dev(graph, torch.int32, "graph", (b.shape[0], None))
        ids, d = _outs(out, nq, k)
        it = torch.empty(nq, dtype=torch.int32, device="cuda")
        ev = torch.empty(nq, dtype=torch.int32, device="cuda") if want_evals else None
        _check(lib.fgpu_graph_search(_dev_ptr(q), nq, _dev_ptr(b), b.shape[0], dim, _dev_ptr(g), g.shape[1], itopk,
                                     width, max_iter, k, seed, _dev_ptr(ids), _dev_ptr(d), _dev_ptr(it), _opt_ptr(ev),
                                     _stream()))
    return (ids, d, it, ev) if want_evals else (ids, d, it)


def fixed_shift(maxabs: float, n: int) -> int:
    return lib.fgpu_fixed_shift(maxabs, n)


def kmeans_update(x, assign, centroids, shift: int, empty_rule: int = 0, stream=None):
    """One deterministic Lloyd update in place on `centroids` (device); returns counts."""
    torch = _torch()
    with _on(stream):
        x = _dev(x, torch.float32, "x", (None, None))
        n, dim = x.shape
        a = _dev(assign, torch.int32, "assign", (n,))
        k = centroids.shape[0]
        _out(centroids, torch.float32, (k, dim), "centroids")
        ws = _workspace(lib.fgpu_kmeans_workspace_bytes(k, dim))
        counts = torch.empty(k, dtype=torch.int32, device="cuda")
        _check(lib.fgpu_kmeans_update(_dev_ptr(x), n, _dev_ptr(a), k, dim, shift, empty_rule, _dev_ptr(centroids),
                                      _dev_ptr(counts), _dev_ptr(ws), _ws_check(ws), _stream()))
    return counts


def kmeans_fit(x, k: int, iters: int, init_mode: int = 0, seed: int = 42, want_assign: bool = True, stream=None):
    torch = _torch()
    with _on(stream):
        x = _dev(x, torch.float32, "x", (None, None))
        n, dim = x.shape
        cent = torch.empty((k, dim), dtype=torch.float32, device="cuda")
        assign = torch.empty(n, dtype=torch.int32, device="cuda") if want_assign else None
        _check(lib.fgpu_kmeans_fit(_dev_ptr(x), n, dim, k, iters, init_mode, seed, _dev_ptr(cent), _opt_ptr(assign),
                                   _stream()))
    return cent, assign


def pq_train(x, assign, centroids, pq_m: int, sample_size: int = 50000, iters: int = 8, stream=None):
    torch = _torch()
    with _on(stream):
        x = _dev(x, torch.float32, "x", (None, None))
        n, dim = x.shape
        a = _dev(assign, torch.int32, "assign", (n,))
        c = _dev(centroids, torch.float32, "centroids", (None, dim))
        if pq_m < 1 or dim % pq_m:
            raise ValueError(f"pq_train: dim {dim} is not a multiple of pq_m {pq_m}")
        cb = torch.empty((pq_m, 256, dim // pq_m), dtype=torch.float32, device="cuda")
        _check(lib.fgpu_pq_train(_dev_ptr(x), n, dim, pq_m, _dev_ptr(a), _dev_ptr(c), sample_size, iters,
                                 _dev_ptr(cb), _stream()))
    return cb


def pq_encode(x, assign, centroids, codebook, fma_mode: int = 1, stream=None):
    """Residual PQ codes (fgpu_pq_encode_form): fma_mode 1 = the device kernel's fused chain
    (kmeans_gpu.cuh:403-445), 0 = the host twin's separately rounded form (pq_utils.h:141-175)."""
    torch = _torch()
    with _on(stream):
        x = _dev(x, torch.float32, "x", (None, None))
        n, dim = x.shape
        a = _dev(assign, torch.int32, "assign", (n,))
        c = _dev(centroids, torch.float32, "centroids", (None, dim))
        cb = _dev(codebook, torch.float32, "codebook", (None, 256, None))
        pq_m = cb.shape[0]
        if pq_m * cb.shape[2] != dim:
            raise ValueError(f"pq_encode: codebook {tuple(cb.shape)} does not cover dim {dim}")
        codes = torch.empty((n, pq_m), dtype=torch.uint8, device="cuda")
        _check(lib.fgpu_pq_encode_form(_dev_ptr(x), n, dim, pq_m, _dev_ptr(a), _dev_ptr(c), _dev_ptr(cb), int(fma_mode),
                                       _dev_ptr(codes), _stream()))
    return codes


def build_ivfpq(x, nlist: int, pq_m: int, kmeans_iters: int = 20, init_mode: int = 0, seed: int = 42,
                pq_iters: int = 8, sample_size: int = 50000, train_rows: int = 0, stream=None):
    """build_global without rebalancing: host arrays (offsets, ids, codes, centroids, codebook).
    train_rows > 0 trains the k-means on the systematic sample of that many rows."""
    with _on(stream):
        x = _dev(x, _torch().float32, "x", (None, None))
        n, dim = x.shape
        if pq_m < 1 or dim % pq_m:
            raise ValueError(f"build_ivfpq: dim {dim} is not a multiple of pq_m {pq_m}")
        offs = np.empty(nlist + 1, np.int32)
        ids = np.empty(n, np.int32)
        codes = np.empty((n, pq_m), np.uint8)
        cent = np.empty((nlist, dim), np.float32)
        cb = np.empty((pq_m, 256, dim // pq_m), np.float32)
        _check(lib.fgpu_build_ivfpq_sampled(_dev_ptr(x), n, dim, nlist, pq_m, train_rows, kmeans_iters, init_mode,
                                            seed, pq_iters, sample_size, _np_ptr(offs), _np_ptr(ids), _np_ptr(codes),
                                            _np_ptr(cent), _np_ptr(cb), _stream()))
    return offs, ids, codes, cent, cb
