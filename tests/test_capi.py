"""CPU checks of libfusiongpu.so that make no device calls: every symbol that
include/fusiongpu.h declares is exported, host-side logic (generator, file
formats, error paths) behaves like the reference's."""
import ctypes
import os
import re

import numpy as np
import pytest

import fusiongpu_amd as fg
import oracle

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "fusiongpu.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(fgpu_[a-z0-9_]+)\s*\(", txt)))


def test_every_declared_symbol_is_exported():
    names = _declared()
    assert len(names) >= 25
    lib = ctypes.CDLL(fg.lib_path)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_mirror_binds_every_symbol():
    assert set(_declared()) <= set(fg._SIGS), set(_declared()) - set(fg._SIGS)


def test_abi_version():
    assert fg.lib.fgpu_abi_version() == 1


@pytest.mark.parametrize("n,k", [(1, 1), (300, 256), (65536, 50000), (65537, 50000), (70001, 256),
                                 (1_000_000, 50000), (3_000_001, 50000)])
def test_pq_sample_prefix_equals_full_shuffle(n, k):
    """fgpu_pq_train draws its sample rows without the n-entry shuffle array
    (only the first k positions are kept); they must equal the oracle's full
    std::shuffle of 0 .. n-1 with mt19937(12345), on both of libstdc++'s
    paths (n <= 65536 takes the paired-draw one)."""
    got = fg.debug_pq_sample(n, k)
    want = oracle.pq_sample(n, k)
    assert np.array_equal(got, want)


def test_generator_matches_oracle_definition():
    for (n, dim, nc, sig, sig2, seed, s) in [(3000, 128, 64, 0.1, None, 1, 0), (500, 96, 16, 0.05, 0.15, 9, 1)]:
        a = fg.gen_gmm(n, dim, nc, seed, set=s, sig_lo=sig, sig_hi=sig2, nthreads=4)
        b = oracle.gen_gmm(n, dim, nc, seed, set=s, sig_lo=sig, sig_hi=sig2)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_ivf_data_round_trip_and_layout(tmp_path):
    rng = np.random.default_rng(0)
    nlist, n, m, dim = 5, 40, 32, 128
    a = rng.integers(0, nlist, n).astype(np.int32)
    codes = rng.integers(0, 256, (n, m)).astype(np.uint8)
    offs, ids, lc = oracle.build_lists(a, nlist, codes)
    cent = rng.standard_normal((nlist, dim)).astype(np.float32)
    p = tmp_path / "ivf_data.bin"
    fg.write_ivf_data(p, offs, ids, lc, cent)
    raw = p.read_bytes()
    # build_global.cu:242-252: i32 total, i32 nlist, offsets, ids, codes, centroids
    assert len(raw) == 8 + 4 * (nlist + 1) + 4 * n + n * m + 4 * nlist * dim
    assert np.frombuffer(raw[:8], np.int32).tolist() == [n, nlist]
    assert np.array_equal(np.frombuffer(raw[8:8 + 4 * (nlist + 1)], np.int32), offs)
    o2, i2, c2, ce2 = fg.read_ivf_data(p, m, dim)
    assert np.array_equal(o2, offs) and np.array_equal(i2, ids) and np.array_equal(c2, lc)
    assert np.array_equal(ce2, cent)
    with pytest.raises(fg.FgpuError) as e:
        fg.read_ivf_data(p, 16, dim)  # wrong geometry -> size mismatch, not a silent misread
    assert e.value.status == 4


def test_fvecs_ivecs_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    v = rng.standard_normal((7, 128)).astype(np.float32)
    p = tmp_path / "x.fvecs"
    fg.write_fvecs(p, v)
    assert np.array_equal(fg.read_fvecs(p, 128), v)
    with pytest.raises(fg.FgpuError):
        fg.read_fvecs(p, 96)  # utils.h:31-34 dimension check
    iv = rng.integers(0, 1000, (4, 10)).astype(np.int32)
    q = tmp_path / "gt.ivecs"
    with open(q, "wb") as f:
        for row in iv:
            f.write(np.int32(10).tobytes() + row.tobytes())
    assert np.array_equal(fg.read_ivecs(q), iv)


@pytest.mark.skipif(oracle.ref_lib() is None, reason="oracle/_ref not built (needs /root/reference)")
def test_fvecs_writer_matches_reference_reader(tmp_path):
    ref = oracle.ref_lib()
    v = np.arange(3 * 128, dtype=np.float32).reshape(3, 128)
    p = tmp_path / "b.fvecs"
    fg.write_fvecs(p, v)
    out = ctypes.POINTER(ctypes.c_float)()
    n = ref.ref_read_fvecs(str(p).encode(), 128, ctypes.byref(out))
    got = np.ctypeslib.as_array(out, shape=(n * 128,)).reshape(n, 128).copy()
    ref.ref_free_f(out)
    assert np.array_equal(got, v)


def test_error_paths_without_device(tmp_path):
    with pytest.raises(fg.FgpuError) as e:
        fg.Index.load(tmp_path / "missing.bin", tmp_path / "cb.bin", 128, 32)
    assert e.value.status == 4
    bad = tmp_path / "short.bin"
    bad.write_bytes(np.array([100, 4], np.int32).tobytes())
    with pytest.raises(fg.FgpuError):
        fg.read_ivf_data(bad, 32, 128)
    assert fg.fixed_shift(1.5, 1 << 20) == oracle.fixed_shift(1.5, 1 << 20)
    assert fg.fixed_shift(0.0, 10) == oracle.fixed_shift(0.0, 10)
