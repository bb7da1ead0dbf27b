"""The K3-scale layer at its full size against the oracle.

Hidden 7168, 384 experts of intermediate 2048, top-16 sigmoid routing,
2x4096 12-bit codes: the decode workload's layer. Sixteen experts have
records and the bias lifts them (as the decode benchmark's cache does), so
every token's sixteen picks are those, in an order its scores set. Decode
on both matvec kernels and a 4-token chunk: picks bit-exact, outputs within
1e-4 of the oracle's moe_layer / moe_chunk; with and without a Q8G shared
expert of intermediate 2048 (whose decode runs inside the router and
combine launches).
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err, routed_share
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module", params=[0, 8], ids=["no-shared", "q8g-shared"])
def k3(request):
    import warp_amd
    ids = tuple(int(i) for i in np.random.default_rng(3).permutation(384)[:16])
    spec = ct.Spec(hidden=7168, inter=2048, experts=384, top_k=16, layers=1, fmt="VQ12", seed=71,
                   shared_bits=request.param, materialize=ids, **BALANCED)
    model = ct.build(spec)
    b = np.zeros(384, np.float32)
    b[list(ids)] = 1.0
    model.layers[0].bias = b
    ctx = open_ctx(model, max_tokens=4, cache_slots=16)
    warp_amd.load_container_model(ctx, model)
    ctx.set_router(0, np.ascontiguousarray(model.layers[0].router, np.float32), b)
    log(f"K3-size layer loaded (shared bits {request.param})")
    yield request.param, model, ctx
    ctx.close()


@pytest.mark.parametrize("path", ["auto", "mfma", "gather"])
def test_k3_decode_full_size(k3, path):
    shared, model, ctx = k3
    ctx.set_matvec_path(path)
    lv = po.LayerView(model, 0)
    worst = 0.0
    try:
        for t in range(3):
            x = np.random.default_rng(100 + t).normal(size=7168).astype(np.float32)
            if t == 0:
                assert routed_share(model, 0, x) > 0.05
            ro, ri, _, _ = lv.moe_layer(x)
            out = empty(7168)
            idx, _ = ctx.moe_decode(0, dev(x), out, want_route=True)
            assert np.array_equal(idx, ri), (t, idx, ri)
            e = rel_err(host(out), ro)
            worst = max(worst, e)
            assert e <= TOL, (t, e)
    finally:
        ctx.set_matvec_path("auto")
    log(f"K3 decode, full size ({path}, shared {shared}): picks bit-exact, worst rel err {worst:.2e}")


def test_k3_chunk_full_size(k3):
    shared, model, ctx = k3
    X = np.random.default_rng(200).normal(size=(4, 7168)).astype(np.float32)
    out, route, _ = ctx.moe_chunk_host(0, X)
    ro, rr, _ = po.LayerView(model, 0).moe_chunk(X)
    assert np.array_equal(route, rr)
    e = rel_err(out, ro)
    assert e <= TOL, e
    log(f"K3 chunk of 4, full size (shared {shared}): routes bit-exact, rel err {e:.2e}")
