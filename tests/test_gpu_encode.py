"""The encoder on the device against the reference's own (src/vq.c).

warp_hip_vq_encode must give the codes of waste_vq_encode bit for bit:
per stage the first minimum of the squared distance summed in dimension
order with unfused fp32 arithmetic, the exact residual feeding the next
stage. Checked against the compiled reference (oracle/_ref) on random
vectors, a duplicated codebook entry (the first copy wins) and vectors equal
to codebook entries; the 4096-entry variant (16-bit codes, beyond the
reference's 8-bit output) against the oracle's restatement. One
warp_hip_vq_lloyd iteration must give the reference's centroids bit for bit
(means summed in double in index order) and its count of non-empty
clusters, with clusters left empty.
"""
import ctypes
import os

import numpy as np
import pytest

from gpu_util import log
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu


def ref_lib():
    if not os.path.exists(po.REF_LIB):
        pytest.skip("compiled reference not built")
    L = ctypes.CDLL(po.REF_LIB)
    L.waste_vq_encode.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
    L.waste_vq_encode.restype = None
    L.waste_vq_lloyd.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int]
    L.waste_vq_lloyd.restype = ctypes.c_int
    return L


def test_encode_matches_reference():
    import warp_amd.hip as wh
    L = ref_lib()
    rng = np.random.default_rng(61)
    S, E, n = 3, 256, 20000
    books = rng.normal(0.0, 1.0, size=(S, E, 8)).astype(np.float32)
    books[0, 40] = books[0, 7]                        # a duplicate: entry 7 must win
    X = rng.normal(0.0, 1.0, size=(n, 8)).astype(np.float32)
    X[:50] = books[0, 7]                              # exactly on the duplicated entry
    X[50:100] = books[0, rng.integers(0, E, 50)]      # exactly on entries
    got = wh.vq_encode(X, books)
    ref = np.empty((n, S), np.uint8)
    L.waste_vq_encode(X.ctypes.data, n, books.ctypes.data, S, E, 8, ref.ctypes.data, 4)
    assert np.array_equal(got, ref), int(np.count_nonzero(got != ref))
    assert (got[:50, 0] == 7).all()
    log(f"vq_encode: {n} vectors x {S} stages of {E} bit-identical to waste_vq_encode")


def test_encode16_matches_oracle():
    import warp_amd.hip as wh
    rng = np.random.default_rng(62)
    S, E, n = 2, 4096, 6000
    books = rng.normal(0.0, 0.5, size=(S, E, 8)).astype(np.float32)
    books[1, 4000] = books[1, 12]
    X = rng.normal(0.0, 1.0, size=(n, 8)).astype(np.float32)
    got = wh.vq_encode(X, books)
    ref = np.empty((n, S), np.uint16)
    po.lib().or_vq_encode(X.ctypes.data, n, books.ctypes.data, S, E, 8, ref.ctypes.data)
    assert got.dtype == np.uint16 and np.array_equal(got, ref), int(np.count_nonzero(got != ref))
    log(f"vq_encode16: {n} vectors x {S} stages of {E} bit-identical to the oracle")


def test_lloyd_matches_reference():
    import warp_amd.hip as wh
    L = ref_lib()
    rng = np.random.default_rng(63)
    n, E = 30000, 256
    X = rng.normal(0.0, 1.0, size=(n, 8)).astype(np.float32)
    C0 = X[rng.permutation(n)[:E]].copy()
    C0[200:] = 1.0e6                                  # far away: these clusters stay empty
    for it in range(3):
        got, ref = C0.copy(), C0.copy()
        live = wh.vq_lloyd(X, got)
        live_ref = L.waste_vq_lloyd(X.ctypes.data, n, ref.ctypes.data, E, 8, 4)
        assert live == live_ref == 200, (live, live_ref)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), it
        C0 = ref
    log(f"vq_lloyd: 3 iterations over {n} vectors, {E} clusters (56 empty) bit-identical to waste_vq_lloyd")
