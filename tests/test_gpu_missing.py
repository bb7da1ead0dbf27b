"""A picked expert that has no resident record and no way to be fetched.

The reference fetches every picked expert before it computes a layer
(src/model.c:2886-2906); a context without a fetch callback cannot, so the
device flags the pick, the layer's output is poisoned with NaN instead of
being computed from a wrong record, and the next synchronising call reports
E_MISSING naming no layer. The flag is sticky until reported, and a later
step whose picks are all resident computes normally (the oracle's result
within the bar). Both decode kernels are covered: the table kernel, whose
gate/up launch routes the token itself, and the decode-then-dot kernel after
the routing launch.
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4
SPEC = dict(hidden=256, inter=128, experts=32, top_k=4, layers=1, fmt="VQ12", seed=61, **BALANCED)
RESIDENT = np.arange(0, 32, 4)                     # experts 0, 4, ..., 28 have records


@pytest.mark.parametrize("path", ["auto", "mfma"])
def test_missing_expert_is_reported(path):
    import warp_amd
    model = ct.build(ct.Spec(materialize=tuple(int(i) for i in RESIDENT), **SPEC))
    lay = model.layers[0]
    router = np.ascontiguousarray(lay.router, np.float32)
    ctx = open_ctx(model, cache_slots=len(RESIDENT))
    try:
        warp_amd.load_container_model(ctx, model)
        ctx.set_matvec_path(path)
        x = np.random.default_rng(3).normal(size=SPEC["hidden"]).astype(np.float32)

        # expert 5 (no record) lifted above everything: it is always picked
        b = np.zeros(SPEC["experts"], np.float32)
        b[RESIDENT] = 1.0
        b[5] = 10.0
        ctx.set_router(0, router, b)
        out = empty(SPEC["hidden"])
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.moe_decode(0, dev(x), out, want_route=True)
        assert ei.value.code == warp_amd.E_MISSING, ei.value
        assert np.isnan(host(out)).all(), "the layer was computed from a missing record"

        # all picks resident again: the flag was cleared when reported
        b[5] = 0.0
        ctx.set_router(0, router, b)
        lay.bias = b
        ro, ri, _, _ = po.LayerView(model, 0).moe_layer(x)
        out = empty(SPEC["hidden"])
        idx, _ = ctx.moe_decode(0, dev(x), out, want_route=True)
        assert np.array_equal(idx, ri), (idx, ri)
        e = rel_err(host(out), ro)
        assert e <= TOL, e
        log(f"[{path}] missing pick reported as E_MISSING with a NaN layer; resident picks after it: rel err {e:.2e}")
    finally:
        ctx.close()
