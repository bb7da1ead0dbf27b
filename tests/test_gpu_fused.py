"""The fused decode launch (k_moe_fused: gate/up, down and combine of a
decode step as work items of one launch) against the same table kernel run
as separate launches, through the C ABI: the outputs, picks and weights
must be identical bit for bit, since the partial sums, their split counts
and every summation order are the same.

Covered: the four float-table formats (VQ3R, VQ2R, the 12-bit format and
its exponent-31 codebook variant), sigmoid and softmax routing, the
residual and a shared expert added by the combine, a latent MoE, the
K3-size layer (hidden 7168, 384 experts, top-16, intermediate 2048), many
launches in a row (the launch leaves its counters zeroed for the next), a
graph replayed with eager work between replays, and a pick without a record
(NaN output, E_MISSING, then a clean launch).
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx

pytestmark = pytest.mark.gpu


def lifted_model(spec_kw, ids, seed):
    model = ct.build(ct.Spec(materialize=tuple(int(i) for i in ids), seed=seed, **spec_kw))
    lay = model.layers[0]
    b = np.zeros(spec_kw["experts"], np.float32) if lay.bias is None else lay.bias.copy()
    b[list(ids)] += 1.0
    lay.bias = b
    return model


def both_paths(ctx, X, resid=None):
    """Decode each row of X with the fused launch and with separate
    launches; returns (fused, separate) outputs and picks."""
    H = X.shape[1]
    res = {}
    for path in ("fused", "auto"):
        ctx.set_matvec_path(path)
        outs, picks = [], []
        for t in range(X.shape[0]):
            out = empty(H)
            idx, w = ctx.moe_decode(0, dev(X[t]), out, want_route=True, resid_dev=None if resid is None
                                    else dev(resid[t]))
            outs.append(host(out).copy())
            picks.append((idx.copy(), w.copy()))
        res[path] = (np.stack(outs), picks)
    ctx.set_matvec_path("auto")
    return res["fused"], res["auto"]


def same_bits(a, b):
    fa, pa = a
    fb, pb = b
    assert np.array_equal(fa.view(np.uint32), fb.view(np.uint32)), float(np.max(np.abs(fa - fb)))
    for (i1, w1), (i2, w2) in zip(pa, pb):
        assert np.array_equal(i1, i2)
        assert np.array_equal(w1.view(np.uint32), w2.view(np.uint32))


CASES = [
    dict(fmt="VQ3R", act=0, shared=0, latent=0),
    dict(fmt="VQ2R", act=1, shared=0, latent=0),
    dict(fmt="VQ12", act=0, shared=8, latent=0),
    dict(fmt="VQ12", act=1, shared=4, latent=0),
    dict(fmt="VQ3R", act=0, shared=8, latent=256),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c['fmt']}-act{c['act']}-sh{c['shared']}-lat{c['latent']}")
def test_fused_equals_launches(case):
    import warp_amd
    E, K, H, I = 64, 8, 1024, 512
    ids = np.random.default_rng(7).permutation(E)[:24]
    kw = dict(hidden=H, inter=I, experts=E, top_k=K, layers=1, fmt=case["fmt"], shared_bits=case["shared"],
              shared_group=32 if case["shared"] == 8 else 128, latent=case["latent"], subnormals=False,
              keep_codes=False, **BALANCED)
    model = lifted_model(kw, ids, seed=200 + len(case["fmt"]) + case["act"])
    ctx = open_ctx(model, router_act=case["act"])
    try:
        warp_amd.load_container_model(ctx, model)
        rng = np.random.default_rng(11)
        X = rng.normal(size=(4, H)).astype(np.float32)
        R = rng.normal(size=(4, H)).astype(np.float32)
        fused, sep = both_paths(ctx, X, R)
        same_bits(fused, sep)
        assert np.all(np.isfinite(fused[0]))
        log(f"fused decode {case}: bit-identical to the separate launches over 4 tokens")
    finally:
        ctx.close()


def test_fused_x31_codebooks():
    """Codebooks with exponent-31 fp16 values take the table kernel's exact
    vector-ALU build in both paths."""
    import warp_amd
    E, K, H, I = 32, 4, 512, 256
    ids = np.arange(E)
    model = lifted_model(dict(hidden=H, inter=I, experts=E, top_k=K, layers=1, fmt="VQ3R", subnormals=False,
                              keep_codes=False, **BALANCED), ids, seed=301)
    raw = model.books_raw.copy()
    raw.reshape(-1)[5] = np.uint16(0x7C00 | 0x12)   # an exponent-31 code value (finite in the reference)
    model.books_raw = raw
    ctx = open_ctx(model)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(5).normal(size=(3, H)).astype(np.float32)
        fused, sep = both_paths(ctx, X)
        same_bits(fused, sep)
        log("fused decode with exponent-31 codebooks: bit-identical to the separate launches")
    finally:
        ctx.close()


def test_fused_k3_size_repeated_and_graph():
    """The K3-size layer: 12 launches in a row, then one captured in a graph
    and replayed 5 times with eager launches between; every output equals
    the separate launches' bit for bit."""
    import warp_amd
    from warp_amd.device import D2D, Graph, copy_async
    ids = np.random.default_rng(3).permutation(384)[:16]
    model = lifted_model(dict(hidden=7168, inter=2048, experts=384, top_k=16, layers=1, fmt="VQ12",
                              subnormals=False, keep_codes=False, **BALANCED), ids, seed=71)
    ctx = open_ctx(model, cache_slots=16)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(21).normal(size=(12, 7168)).astype(np.float32)
        fused, sep = both_paths(ctx, X)
        same_bits(fused, sep)
        xs = [dev(x) for x in X]
        stage, out = empty(7168), empty(7168)
        ctx.set_matvec_path("fused")
        g = Graph(ctx.stream, lambda: ctx.moe_decode(0, stage, out))
        try:
            for rep in range(5):
                ctx.moe_decode(0, xs[1 + rep], empty(7168))           # eager work between replays
                copy_async(stage.ptr, xs[rep].ptr, 7168 * 4, D2D, ctx.stream)
                g.launch()
                ctx.sync()
                assert np.array_equal(host(out).view(np.uint32), fused[0][rep].view(np.uint32)), rep
        finally:
            g.free()
        log("fused K3-size decode: 12 launches and 5 graph replays bit-identical to the separate launches")
    finally:
        ctx.close()


def test_fused_missing_pick_then_clean():
    """A pick without a record (no fetch function): the fused launch writes
    NaN, the next synchronising call reports E_MISSING, and the launch
    after that (all picks resident) is exact again."""
    import warp_amd
    E, K, H, I = 32, 4, 512, 256
    ids = np.arange(8)
    model = lifted_model(dict(hidden=H, inter=I, experts=E, top_k=K, layers=1, fmt="VQ3R", subnormals=False,
                              keep_codes=False, **BALANCED), ids, seed=41)
    ctx = open_ctx(model)
    try:
        warp_amd.load_container_model(ctx, model)
        x = np.random.default_rng(2).normal(size=H).astype(np.float32)
        ref = empty(H)
        ctx.moe_decode(0, dev(x), ref)
        ctx.sync()
        ctx.set_matvec_path("fused")
        b = model.layers[0].bias.copy()
        b[20] = 50.0                                     # expert 20 has no record
        ctx.set_router(0, np.ascontiguousarray(model.layers[0].router, np.float32), b)
        out = empty(H)
        ctx.moe_decode(0, dev(x), out)
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.sync()
        assert ei.value.code == warp_amd.E_MISSING
        assert np.all(np.isnan(host(out)))
        ctx.set_router(0, np.ascontiguousarray(model.layers[0].router, np.float32), model.layers[0].bias)
        out2 = empty(H)
        ctx.moe_decode(0, dev(x), out2)
        ctx.sync()
        ctx.set_matvec_path("auto")
        assert np.array_equal(host(out2).view(np.uint32), host(ref).view(np.uint32))
        log("fused decode: missing pick -> NaN + E_MISSING, then exact again")
    finally:
        ctx.close()
