"""The real K3 shape (the reference's docs/K3.md:33-46) against the oracle.

Hidden 7168, 896 routed experts with a Stable LatentMoE: the experts run on
a 3584-wide projection of the hidden state (routed_expert_down_proj), with
moe_intermediate 3072, top-16 sigmoid routing with a bias, RMS norm and
routed_expert_up_proj after the weighted sum (src/model.c:2789-2795,
2913-2921), two shared experts (intermediate 2 x 3072) on the hidden
state; VQ3R records, Q8G projections and shared experts. Above 512 experts
the routing is a launch of its own rather than part of the gate/up launch.
Twenty-four experts have records and the bias lifts them, so every token's
sixteen picks are among those. Decode on both matvec kernels and a 4-token
chunk: picks bit-exact, outputs within 1e-4 of max|ref| of the oracle's
moe_layer / moe_chunk.
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err, routed_share
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4
E = 896


@pytest.fixture(scope="module")
def k3real():
    import warp_amd
    ids = tuple(int(i) for i in np.random.default_rng(5).permutation(E)[:24])
    spec = ct.Spec(hidden=7168, inter=3072, experts=E, top_k=16, layers=1, fmt="VQ3R", seed=81, latent=3584,
                   latent_norm=True, shared_bits=8, shared_group=32, n_shared=2, routed_scale=2.827,
                   subnormals=False, keep_codes=False, materialize=ids, **BALANCED)
    model = ct.build(spec)
    b = np.zeros(E, np.float32)
    b[list(ids)] = 1.0
    model.layers[0].bias = b
    ctx = open_ctx(model, max_tokens=4, cache_slots=24)
    warp_amd.load_container_model(ctx, model)
    log("real K3 layer loaded: 896 experts, latent 3584, inter 3072, two shared experts")
    yield model, ctx
    ctx.close()


@pytest.mark.parametrize("path", ["auto", "mfma", "gather"])
def test_k3_real_decode(k3real, path):
    model, ctx = k3real
    ctx.set_matvec_path(path)
    lv = po.LayerView(model, 0)
    worst = 0.0
    try:
        for t in range(3):
            x = np.random.default_rng(300 + t).normal(size=7168).astype(np.float32)
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
    log(f"real K3 decode ({path}): picks bit-exact, worst rel err {worst:.2e}")


def test_k3_real_chunk(k3real):
    model, ctx = k3real
    X = np.random.default_rng(400).normal(size=(4, 7168)).astype(np.float32)
    out, route, _ = ctx.moe_chunk_host(0, X)
    ro, rr, _ = po.LayerView(model, 0).moe_chunk(X)
    assert np.array_equal(route, rr)
    e = rel_err(out, ro)
    assert e <= TOL, e
    log(f"real K3 chunk of 4: routes bit-exact, rel err {e:.2e}")
