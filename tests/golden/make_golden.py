"""Writes tests/golden/ref_pq.npz from the reference's own CPU code.

Runs oracle/_ref/libref.so -- /root/reference/pq_utils.h compiled as-is by
oracle/Makefile -- on small seeded inputs and stores its outputs.  Inputs are
regenerated from the seeds below with numpy's PCG64, so only outputs are
stored.  Run from the repo root:  python tests/golden/make_golden.py
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import ref_lib  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "ref_pq.npz")


def inputs():
    """Seeded inputs shared by make_golden.py and the tests that read the fixture."""
    rng = np.random.default_rng(20241201)
    km_data = rng.standard_normal((700, 4)).astype(np.float32)
    n, nlist = 600, 12
    x = (rng.standard_normal((n, 128)) * 0.3).astype(np.float32)
    cent = rng.standard_normal((nlist, 128)).astype(np.float32) * 0.5
    assign = rng.integers(0, nlist, n).astype(np.int32)
    x += cent[assign]
    return km_data, x, cent.astype(np.float32), assign


def main():
    ref = ref_lib()
    if ref is None:
        sys.exit("oracle/_ref/libref.so not built (needs /root/reference); run make -C oracle")
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    km_data, x, cent, assign = inputs()
    km_out = np.empty((256, 4), np.float32)
    ref.ref_run_kmeans_pq_fast(P(km_data), km_data.shape[0], 4, 256, 1234, 6, P(km_out))
    cb = np.empty((32, 256, 4), np.float32)
    ref.ref_train_residual_pq_codebooks(P(x), x.shape[0], P(assign), P(cent), cent.shape[0], 500, 5, P(cb))
    codes = np.empty((x.shape[0], 32), np.uint8)
    ref.ref_encode_residuals_to_pq(P(x), x.shape[0], P(assign), P(cent), cent.shape[0], P(cb), P(codes))
    np.savez_compressed(OUT, kmeans_fast=km_out, codebook=cb, codes=codes,
                        note=np.array("outputs of /root/reference/pq_utils.h (run_kmeans_pq_fast seed 1234 iters 6; "
                                      "train_residual_pq_codebooks sample 500 iters 5; encode_residuals_to_pq)"))
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
