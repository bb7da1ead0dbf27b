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


@pytest.mark.parametrize("path", ["auto", "mfma", "gather"])
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


def test_refused_device_record_leaves_the_cache_as_it_was():
    """warp_hip_put_expert_dev checks the header of a record already in
    device memory before it touches a slot. A bad header over a resident
    expert is refused (E_HEADER) and the resident record keeps serving
    (output bit-identical to before); a bad header for an expert without a
    record is refused and, with no fetch function, selecting that expert
    later reports E_MISSING with a NaN layer, not a finite output from
    whatever sat in a slot."""
    import warp_amd
    model = ct.build(ct.Spec(materialize=tuple(int(i) for i in RESIDENT), **SPEC))
    lay = model.layers[0]
    router = np.ascontiguousarray(lay.router, np.float32)
    ctx = open_ctx(model, cache_slots=len(RESIDENT) + 1)
    try:
        warp_amd.load_container_model(ctx, model)
        x = np.random.default_rng(5).normal(size=SPEC["hidden"]).astype(np.float32)
        b = np.zeros(SPEC["experts"], np.float32)
        b[RESIDENT] = 1.0
        b[8] = 10.0                                   # resident expert 8 always picked
        ctx.set_router(0, router, b)
        before = empty(SPEC["hidden"])
        idx0, _ = ctx.moe_decode(0, dev(x), before, want_route=True)
        assert 8 in idx0
        good = np.frombuffer(lay.records[8], np.uint8).copy()
        bad = good.copy()
        bad[0] ^= 0xFF                                # magic broken
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.put_expert_dev(0, 8, dev(bad))
        assert ei.value.code == warp_amd.E_HEADER, ei.value
        after = empty(SPEC["hidden"])
        idx1, _ = ctx.moe_decode(0, dev(x), after, want_route=True)
        assert np.array_equal(idx0, idx1)
        assert np.array_equal(host(before).view(np.uint32), host(after).view(np.uint32))
        # expert 5 has no record: its bad header is refused, and picking it is E_MISSING
        bad5 = good.copy()
        bad5[6:8] = np.frombuffer(np.uint16(5).tobytes(), np.uint8)   # identity of expert 5
        bad5[4:6] = np.frombuffer(np.uint16(7).tobytes(), np.uint8)   # ... but of layer 7
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.put_expert_dev(0, 5, dev(bad5))
        assert ei.value.code == warp_amd.E_HEADER, ei.value
        assert not ctx.resident(0, 5)
        b[5] = 20.0
        ctx.set_router(0, router, b)
        out = empty(SPEC["hidden"])
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.moe_decode(0, dev(x), out, want_route=True)
        assert ei.value.code == warp_amd.E_MISSING, ei.value
        assert np.isnan(host(out)).all()
        # a good device record for expert 8 replaces the resident one in place
        ctx.put_expert_dev(0, 8, dev(good))
        b[5] = 0.0
        ctx.set_router(0, router, b)
        again = empty(SPEC["hidden"])
        ctx.moe_decode(0, dev(x), again)
        assert np.array_equal(host(before).view(np.uint32), host(again).view(np.uint32))
        log("put_expert_dev: refused headers leave the cache intact; a refused new expert stays missing")
    finally:
        ctx.close()
