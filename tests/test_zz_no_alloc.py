"""The allocation-free encoder variant (warp_hip_vq_encode_dev_noalloc)
against the encoder with a caller workspace (warp_hip_vq_encode_dev),
through the C ABI: codes bit-identical on two calls in a row on one device,
the second smaller than the first (the shared scratch keeps the first
call's rows, which the second must not read), for 3 x 256 and 2 x 4096
codebooks; a single stage of any size (no scratch used); more vectors than
the scratch holds refused with E_ARG."""

import numpy as np
import pytest

from gpu_util import log

pytestmark = pytest.mark.gpu

def encode_both(X, books, stream=None):
    import warp_amd.hip as wh
    from warp_amd.device import Buf, synchronize
    n = X.shape[0]
    S, E, _ = books.shape
    xd, bd = Buf.of(X), Buf.of(books)
    resid = Buf.empty((n, 8))
    c_ws, c_na = Buf.empty((n, S), np.uint16), Buf.empty((n, S), np.uint16)
    assert wh.lib().warp_hip_vq_encode_dev(xd.ptr, n, bd.ptr, S, E, resid.ptr, c_ws.ptr, stream) == 0
    assert wh.lib().warp_hip_vq_encode_dev_noalloc(xd.ptr, n, bd.ptr, S, E, c_na.ptr, stream) == 0
    synchronize()
    return c_ws.numpy(), c_na.numpy()

@pytest.mark.parametrize("S,E", [(3, 256), (2, 4096)])
def test_noalloc_encoder_equals_workspace_encoder(S, E):
    import warp_amd.hip as wh
    rng = np.random.default_rng(S * 100 + E)
    books = rng.standard_normal((S, E, 8)).astype(np.float32)
    maxn = 1 << 19
    for n in (maxn, 12_345):                      # the full scratch, then a smaller call
        X = rng.standard_normal((n, 8)).astype(np.float32)
        a, b = encode_both(X, books)
        assert np.array_equal(a, b), (n, int(np.count_nonzero(a != b)))
        assert a.max() < E and len(np.unique(a[:, 0])) > min(E, n) // 4
    # one stage: no scratch, any size
    X = rng.standard_normal((maxn + 7, 8)).astype(np.float32)
    a, b = encode_both(X, books[:1])
    assert np.array_equal(a, b)
    # beyond the scratch with stages > 1: refused before anything runs
    from warp_amd.device import Buf
    xd, bd, cd = Buf.empty((maxn + 1, 8)), Buf.of(books), Buf.empty((maxn + 1, S), np.uint16)
    assert wh.lib().warp_hip_vq_encode_dev_noalloc(xd.ptr, maxn + 1, bd.ptr, S, E, cd.ptr, None) == wh.E_ARG
    log(f"noalloc encoder {S}x{E}: codes bit-identical to the workspace encoder on {maxn} then 12,345 vectors; "
        f"one stage of {maxn + 7}; {maxn + 1} vectors refused")
