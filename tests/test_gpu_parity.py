"""Parity of the HIP path (through the C ABI) with the oracle, on the same
synthetic container bytes.

Bars: decoded weights, code unpacking and expert selection bit-exact;
VQ4P (whose reference arithmetic is integer plus a fixed float order) and
the strict router bit-exact; everything else max|d|/max|ref| <= 1e-4 with
fp32 accumulation.
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err, routed_share
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4
FMTS = ["VQ3R", "VQ2R", "VQ4P", "VQ12"]


def small_spec(fmt, **kw):
    base = dict(hidden=128, inter=64, experts=8, top_k=2, layers=2, fmt=fmt, seed=7, **BALANCED)
    base.update(kw)
    return ct.Spec(**base)


@pytest.fixture(scope="module", params=FMTS)
def loaded(request):
    import warp_amd
    fmt = request.param
    model = ct.build(small_spec(fmt))
    ctx = open_ctx(model, max_tokens=16)
    warp_amd.load_container_model(ctx, model)
    log(f"[{fmt}] context loaded, rec_bytes {model.rec_bytes}")
    yield fmt, model, ctx
    ctx.close()


def test_decode_weights_bitexact(loaded):
    fmt, model, ctx = loaded
    spec = model.spec
    books = po.books_flat(model.books_raw)
    for L in range(spec.layers):
        for e in (0, spec.experts - 1):
            rec = ctx.resident(L, e)
            assert rec
            for kind in range(3):
                M, N = (spec.inter, spec.hidden) if kind < 2 else (spec.hidden, spec.inter)
                W = empty((M, N))
                ctx.decode_weights(L, kind, rec, W)
                r = np.frombuffer(model.layers[L].records[e], np.uint8)
                hdr = np.frombuffer(model.layers[L].records[e][:48], np.uint32)
                off = int(hdr[5 + kind])
                corr = int(hdr[8])
                soff = [0, spec.inter, 2 * spec.inter][kind]
                scale = r[corr + 2 * soff: corr + 2 * (soff + M)].view(np.uint16)
                S = ct.FMT_STAGES[fmt]
                Wr = po.decode_weights(fmt, r[off:].copy(), scale.copy(), books, L * 3 * S + kind * S, M, N)
                assert np.array_equal(host(W).view(np.uint32), Wr.view(np.uint32)), (L, e, kind)
    log(f"[{fmt}] decoded weights bit-exact")


@pytest.mark.parametrize("path", ["auto", "mfma", "fused"])
def test_vq_matvec(loaded, path):
    fmt, model, ctx = loaded
    spec = model.spec
    ctx.set_matvec_path(path)
    S = {"VQ3R": 3, "VQ2R": 2, "VQ4P": 4, "VQ12": 2}[fmt]
    bT = po.books_T(model.books_raw)
    rng = np.random.default_rng(3)
    for L in range(spec.layers):
        for e in range(0, spec.experts, 3):
            rec = ctx.resident(L, e)
            r = np.frombuffer(model.layers[L].records[e], np.uint8)
            hdr = np.frombuffer(model.layers[L].records[e][:48], np.uint32)
            for kind in range(3):
                M, N = (spec.inter, spec.hidden) if kind < 2 else (spec.hidden, spec.inter)
                x = rng.normal(size=N).astype(np.float32)
                y = empty(M)
                ctx.vq_matvec(L, kind, rec, dev(x), y)
                off, corr = int(hdr[5 + kind]), int(hdr[8])
                soff = [0, spec.inter, 2 * spec.inter][kind]
                scale = r[corr + 2 * soff: corr + 2 * (soff + M)].view(np.uint16).copy()
                yr = po.vq_matvec(fmt, r[off:].copy(), scale, x, bT, L * 3 * S + kind * S, M, N)
                yg = host(y)
                if fmt == "VQ4P":
                    assert np.array_equal(yg, yr), (L, e, kind, rel_err(yg, yr))
                else:
                    assert rel_err(yg, yr) <= TOL, (L, e, kind, rel_err(yg, yr))
    ctx.set_matvec_path("auto")
    log(f"[{fmt}] vq_matvec ({path}) within bar")


def test_router_strict_and_route(loaded):
    import warp_amd
    fmt, model, ctx0 = loaded
    spec = model.spec
    ctx = open_ctx(model, max_tokens=16, router_strict=True)
    warp_amd.load_container_model(ctx, model)
    rng = np.random.default_rng(11)
    T = 16
    for L in range(spec.layers):
        X = rng.normal(size=(T, spec.hidden)).astype(np.float32)
        lg = empty((T, spec.experts))
        ctx.router_logits(L, dev(X), T, lg)
        W = model.layers[L].router
        ref = np.array([[po.lib().or_dotf(W[e].ctypes.data, X[t].ctypes.data, spec.hidden)
                         for e in range(spec.experts)] for t in range(T)], np.float32)
        assert np.array_equal(host(lg), ref), "strict router logits are not bit-exact"
        # selection and weights on identical logits
        idx = empty((T, spec.top_k), np.int32)
        w = empty((T, spec.top_k))
        ctx.route(L, dev(ref), T, idx, w)
        for t in range(T):
            ri, rw, _ = po.route(ref[t], model.layers[L].bias, spec.top_k, 0, int(spec.renorm), spec.routed_scale)
            assert np.array_equal(host(idx)[t], ri)
            assert np.array_equal(host(w)[t], rw), (host(w)[t], rw)
    ctx.close()
    log(f"[{fmt}] strict router bit-exact, selection and weights bit-exact")


@pytest.mark.parametrize("path", ["auto", "mfma", "gather"])
def test_moe_decode(loaded, path):
    fmt, model, ctx = loaded
    spec = model.spec
    ctx.set_matvec_path(path)
    rng = np.random.default_rng(5)
    worst = 0.0
    for L in range(spec.layers):
        lv = po.LayerView(model, L)
        for t in range(6):
            x = rng.normal(size=spec.hidden).astype(np.float32)
            if t == 0:
                share = routed_share(model, L, x)
                assert share > 0.05, f"the routed experts are {share:.1e} of the output: test not sensitive"
            out = empty(spec.hidden)
            idx, w = ctx.moe_decode(L, dev(x), out, want_route=True)
            ro, ri, rw, _ = lv.moe_layer(x)
            assert np.array_equal(idx, ri), (idx, ri)
            e = rel_err(host(out), ro)
            worst = max(worst, e)
            assert e <= TOL, (L, t, e)
    ctx.set_matvec_path("auto")
    log(f"[{fmt}] moe_decode ({path}) worst rel err {worst:.2e}")


def test_moe_decode_host_matches_device(loaded):
    fmt, model, ctx = loaded
    x = np.random.default_rng(9).normal(size=model.spec.hidden).astype(np.float32)
    out = empty(model.spec.hidden)
    ctx.moe_decode(1, dev(x), out)
    oh, _ = ctx.moe_decode_host(1, x)
    assert np.array_equal(host(out), oh)


def test_moe_chunk(loaded):
    fmt, model, ctx = loaded
    spec = model.spec
    rng = np.random.default_rng(21)
    for L in range(spec.layers):
        lv = po.LayerView(model, L)
        X = rng.normal(size=(13, spec.hidden)).astype(np.float32)
        out, route, rw = ctx.moe_chunk_host(L, X)
        ro, rr, rrw = lv.moe_chunk(X)
        assert np.array_equal(route, rr)
        e = rel_err(out, ro)
        assert e <= TOL, (L, e)
        log(f"[{fmt}] moe_chunk L{L} rel err {e:.2e}")


def test_router_batch_on_matrix_cores():
    """Batches of 16 tokens or more take the fp32 matrix-core router. Its
    logits are within the fp32 summation bound of a float64 product
    (|d| <= H * 2^-24 * sum|w x|); a token's logits do not depend on its
    place in the batch or on the batch size (bit for bit); and they select
    the same experts as the one-token router, whose sum runs in another
    order. Token and expert counts are not multiples of the 16 x 16 block."""
    import warp_amd
    spec = ct.Spec(hidden=256, inter=64, experts=40, top_k=4, layers=1, fmt="VQ3R", seed=17, **BALANCED)
    model = ct.build(spec)
    ctx = open_ctx(model, max_tokens=64)
    try:
        warp_amd.load_container_model(ctx, model)
        rng = np.random.default_rng(19)
        X = rng.normal(size=(45, spec.hidden)).astype(np.float32)
        W = model.layers[0].router
        lg = empty((45, spec.experts))
        ctx.router_logits(0, dev(X), 45, lg)
        got = host(lg)
        ref = X.astype(np.float64) @ W.astype(np.float64).T
        bound = spec.hidden * 2.0 ** -24 * (np.abs(X).astype(np.float64) @ np.abs(W).astype(np.float64).T)
        assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) / bound))
        perm = rng.permutation(45)[:17]
        lg2 = empty((17, spec.experts))
        ctx.router_logits(0, dev(np.ascontiguousarray(X[perm])), 17, lg2)
        assert np.array_equal(host(lg2).view(np.uint32), got[perm].view(np.uint32)), "batch place changed a logit"
        out = empty((45, spec.hidden))
        route, _ = ctx.moe_chunk(0, dev(X), out, 45, want_route=True)
        for t in range(0, 45, 4):
            o = empty(spec.hidden)
            idx, _ = ctx.moe_decode(0, dev(X[t]), o, want_route=True)
            assert np.array_equal(idx, route[t]), t
        log(f"batch router: within the fp32 bound of float64, batch-place invariant, decode picks agree")
    finally:
        ctx.close()


@pytest.mark.parametrize("T", [1, 16, 48])
def test_moe_chunk_sizes(T):
    """A chunk of one token, of exactly the batch router's threshold, and of
    the context's max_tokens (48): routes bit-exact and outputs within the
    bar against the oracle's moe_chunk, a layer with a Q8G shared expert in
    the 12-bit format; one token past max_tokens is refused."""
    import warp_amd
    spec = ct.Spec(hidden=256, inter=128, experts=24, top_k=4, layers=1, fmt="VQ12", seed=43, **BALANCED)
    model = ct.build(spec)
    ctx = open_ctx(model, max_tokens=48)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(47 + T).normal(size=(T, spec.hidden)).astype(np.float32)
        out, route, rw = ctx.moe_chunk_host(0, X)
        ro, rr, rrw = po.LayerView(model, 0).moe_chunk(X)
        assert np.array_equal(route, rr)
        e = rel_err(out, ro)
        assert e <= TOL, e
        if T == 48:
            with pytest.raises(warp_amd.WarpHipError) as ei:
                ctx.moe_chunk_host(0, np.zeros((49, spec.hidden), np.float32))
            assert ei.value.code == warp_amd.E_ARG, ei.value
        log(f"moe_chunk T={T}: routes bit-exact, rel err {e:.2e}")
    finally:
        ctx.close()


@pytest.mark.parametrize("bits,group,hidden,inter", [(8, 32, 160, 96), (4, 128, 256, 128), (8, 64, 192, 320)])
def test_moe_chunk_shared_on_matrix_cores(bits, group, hidden, inter):
    """The chunk's shared expert on the matrix cores (gate and up in one
    launch, 64-row x 64-token tiles, weights staged 128 columns at a time):
    Q8G and Q4G, groups of 32, 64 and 128, shapes that fill neither a tile
    (96, 128, 160, 192, 256 and 320 rows; 40 tokens) nor always a slab (96,
    160, 192 and 320 columns). The shared expert's scales are the default
    0.002-0.02, so it dominates the output and its error is what the bar
    sees. Routes bit-exact, output within the bar against the oracle."""
    import warp_amd
    spec = ct.Spec(hidden=hidden, inter=inter, experts=8, top_k=2, layers=1, fmt="VQ12", seed=53 + bits + group,
                   shared_bits=bits, shared_group=group, book_std=0.3)
    model = ct.build(spec)
    ctx = open_ctx(model, max_tokens=48)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(59).normal(size=(40, hidden)).astype(np.float32)
        out, route, _ = ctx.moe_chunk_host(0, X)
        ro, rr, _ = po.LayerView(model, 0).moe_chunk(X)
        assert np.array_equal(route, rr)
        e = rel_err(out, ro)
        assert e <= TOL, e
        log(f"shared expert Q{bits}G group {group}, {inter}x{hidden}: rel err {e:.2e}")
    finally:
        ctx.close()


def test_moe_chunk_many_pairs():
    """600 tokens x top-16 of 64 experts: 9,600 pairs, more than the grouping
    keeps in registers (8 per thread of its 1,024), so its looping path
    runs; routes bit-exact and outputs within the bar against the oracle."""
    import warp_amd
    spec = ct.Spec(hidden=64, inter=32, experts=64, top_k=16, layers=1, fmt="VQ12", seed=61, **BALANCED)
    model = ct.build(spec)
    ctx = open_ctx(model, max_tokens=600)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(67).normal(size=(600, spec.hidden)).astype(np.float32)
        out, route, _ = ctx.moe_chunk_host(0, X)
        ro, rr, _ = po.LayerView(model, 0).moe_chunk(X)
        assert np.array_equal(route, rr)
        e = rel_err(out, ro)
        assert e <= TOL, e
        log(f"moe_chunk of 600 tokens x top-16 of 64: routes bit-exact, rel err {e:.2e}")
    finally:
        ctx.close()
