"""Certified selection: decode picks bit-identical to the reference's on
planted near-ties, by construction rather than by luck.

The reference ranks experts by sigmoid scores of logits summed sequentially
in fp32 (dotf, src/model.c:155-160; top-k src/model.c:2727-2742). Here 24
router rows are scaled so that their exact logits (float64 sums of the fp32
products) all lie within one ulp of -8 of each other, while the sequential
sum's rounding moves each by several ulps: the order of the cluster, and
which 8 of its 24 rows are picked, is decided by fp32 rounding alone. The
other experts sit near -20. Near -8 the sigmoid keeps those differences
(the score's ulp is far below one logit ulp's effect), and the bias is zero,
so the biased scores keep them too.

The default decode certifies: the router launch bounds each logit's
distance from the reference's sequential sum, and the routing recomputes,
in the reference's order, every row whose bounds leave the picks or their
order open. Checked on the table kernel's fused routing (auto), on the
routing launch (the decode-then-dot path, and above 512 experts), and on the
one-launch decode, against the oracle's sequential router: picks and order
identical, outputs within 1e-4 of max|ref|. The plain fast logits
(router_fast) must get some token's picks wrong on the same inputs, which
shows the inputs do decide on rounding. A tie case: 80 identical rows tie
exactly (more than the 64 survivors the picking's ranking takes in one pass,
so its picking loop runs), and the lowest ids win.
"""
import math

import numpy as np
import pytest

import container as ct
from gpu_util import dev, empty, host, log, open_ctx, rel_err
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4
H = 2048


def exact_logits(W, x):
    """float64-exact logits: fsum of the fp32 products (each exact in double)."""
    P = W.astype(np.float64) * x.astype(np.float64)
    return np.array([math.fsum(r) for r in P])


def plant(rng, E, x, cluster, level=-8.0, rest=-20.0, copies=False):
    """Router rows whose exact logits are level (within a fraction of an ulp)
    for the cluster ids and about rest for the others."""
    W = np.empty((E, H), np.float32)
    base = None
    for e in range(E):
        while True:
            r = rng.normal(0.0, 0.02, H).astype(np.float32)
            d = float(np.dot(r.astype(np.float64), x.astype(np.float64)))
            if abs(d) > 0.3:
                break
        want = level if e in cluster else rest + rng.uniform(-1.0, 1.0)
        w = (r.astype(np.float64) * (want / d)).astype(np.float32)
        # the scaled row's own rounding moved its logit: put the residual
        # into the columns of the largest inputs, one at a time
        for k in np.argsort(-np.abs(x))[:4]:
            res = want - exact_logits(w[None], x)[0]
            w[k] = np.float32(float(w[k]) + res / float(x[k]))
        W[e] = w
        if copies and e in cluster:
            if base is None:
                base = W[e].copy()
            W[e] = base
    return W


def seq_logits(W, x):
    """The reference's dotf for every row (src/model.c:155-160): fp32
    products, added one at a time in index order, unfused (numpy's float32
    operations round to nearest, as the reference's do)."""
    P = (W * x[None, :]).astype(np.float32)
    acc = np.zeros(W.shape[0], np.float32)
    for k in range(W.shape[1]):
        acc = (acc + P[:, k]).astype(np.float32)
    return acc


def build(E, K, cluster, seed, copies=False):
    spec = ct.Spec(hidden=H, inter=64, experts=E, top_k=K, layers=1, fmt="VQ3R", seed=seed, bias=False,
                   shared_bits=0, renorm=True, routed_scale=1.0, subnormals=False, keep_codes=False,
                   materialize=tuple(sorted(cluster)), book_std=0.3)
    return ct.build(spec)


def decode_case(model, ctx, x, paths):
    lv = po.LayerView(model, 0)
    ro, ri, rw, rl = lv.moe_layer(x)
    got = {}
    for path in paths:
        ctx.set_matvec_path(path)
        out = empty(H)
        idx, w = ctx.moe_decode(0, dev(x), out, want_route=True)
        got[path] = (idx, rel_err(host(out), ro), w)
    ctx.set_matvec_path("auto")
    return ri, rl, got, rw


@pytest.mark.parametrize("E", [64, 100, 640])
def test_certified_picks_on_planted_near_ties(E):
    # (100: rows the certifying block polls in a partial last pass, and masks
    # of a last 64-expert word that is not full)
    K, n_tok = 8, 4
    rng = np.random.default_rng(900 + E)
    cluster = set(int(i) for i in rng.permutation(E)[:24])
    model = build(E, K, cluster, seed=31 + E)
    ctx = open_ctx(model)
    fast = open_ctx(model, router_fast=True)
    import warp_amd
    paths = ("auto", "mfma", "fused", "gather") if E <= 512 else ("auto", "mfma", "gather")
    fast_wrong = 0
    try:
        for t in range(n_tok):
            x = rng.normal(size=H).astype(np.float32)
            W = plant(rng, E, x, cluster)
            ex = exact_logits(W, x)
            cl = np.array(sorted(cluster))
            # the planted gaps: every exact cluster logit within one ulp of -8
            assert np.ptp(ex[cl]) < np.spacing(np.float32(8.0)), np.ptp(ex[cl])
            model.layers[0].router = W
            for c in (ctx, fast):
                warp_amd.load_container_model(c, model, records=(t == 0))
            ri, rl, got, rw = decode_case(model, ctx, x, paths)
            # the reference's logits spread over several ulps: rounding decides
            spread = np.ptp(rl[cl].astype(np.float64)) / float(np.spacing(np.float32(8.0)))
            assert set(ri.tolist()) <= cluster
            for path, (idx, err, w) in got.items():
                assert np.array_equal(idx, ri), (t, path, idx, ri)
                assert err <= TOL, (t, path, err)
                # every pick was recomputed: its score is the reference's, and so
                # the weights (the same sum in the same order) are the reference's
                assert np.array_equal(w, rw), (t, path, w, rw)
            fi = decode_case(model, fast, x, ("auto",))[2]["auto"][0]
            fast_wrong += int(not np.array_equal(fi, ri))
            log(f"E={E} token {t}: reference logits of the cluster spread over {spread:.1f} ulps; "
                f"certified picks identical on {', '.join(paths)}; fast picks "
                f"{'identical' if np.array_equal(fi, ri) else 'different'}")
        st = ctx.route_stats()
    finally:
        ctx.close()
        fast.close()
    log(f"E={E}: fast logits wrong on {fast_wrong} of {n_tok} tokens; route stats {st}")
    assert fast_wrong >= 1
    assert st["certified"] >= n_tok * len(paths) and st["recomputed"] >= n_tok and st["rows"] >= n_tok * 24


def test_certified_exact_ties_take_lowest_ids():
    E, K = 256, 8
    rng = np.random.default_rng(77)
    cluster = set(range(40, 120))
    model = build(E, K, cluster, seed=5, copies=True)
    ctx = open_ctx(model)
    import warp_amd
    try:
        x = rng.normal(size=H).astype(np.float32)
        model.layers[0].router = plant(rng, E, x, cluster, copies=True)
        warp_amd.load_container_model(ctx, model)
        ri, rl, got, rw = decode_case(model, ctx, x, ("auto", "mfma", "fused", "gather"))
        assert list(ri) == list(range(40, 48)), ri            # exact ties: the lowest ids, in order
        for path, (idx, err, w) in got.items():
            assert np.array_equal(idx, ri), (path, idx, ri)
            assert err <= TOL, (path, err)
            assert np.array_equal(w, rw), (path, w, rw)
        st = ctx.route_stats()
    finally:
        ctx.close()
    log(f"80 tied rows: picks {list(ri)} on every path; route stats {st}")
    assert st["rows"] >= 3 * 80


@pytest.mark.parametrize("H_, scale", [(7168, 1.0), (2304, 1.0), (2048, 1.0), (1056, 1.0), (2304, 40.0)])
def test_router_bounds_hold_the_reference_scores(H_, scale):
    """The certified router's bounds (warp_hip_router_cert) against the
    reference's biased scores: the oracle's sequential logits, its sigmoid
    (glibc expf) and the bias, for every expert of several tokens. Widths:
    the staged kernels at 7168 / 2304 / 2048, the general kernel at 1000,
    and logits beyond +-30 (scale 40), where the bounds come from the
    reference's own expf."""
    E, K = 256, 8
    spec = ct.Spec(hidden=H_, inter=64, experts=E, top_k=K, layers=1, fmt="VQ3R", seed=3, bias=True,
                   shared_bits=0, renorm=True, routed_scale=1.0, subnormals=False, keep_codes=False,
                   materialize=(0,), book_std=0.3)
    model = ct.build(spec)
    model.layers[0].router = (model.layers[0].router * np.float32(scale)).astype(np.float32)
    ctx = open_ctx(model)
    import warp_amd
    worst = 0.0
    try:
        warp_amd.load_container_model(ctx, model, records=False)
        rng = np.random.default_rng(H_)
        P_all = model.layers[0].router
        for t in range(6):
            x = rng.normal(size=H_).astype(np.float32)
            rl = seq_logits(P_all, x)
            _, _, sc = po.route(rl, model.layers[0].bias, K)
            ref = (sc + model.layers[0].bias).astype(np.float32)
            out = empty(4 * E)
            ctx.router_cert(0, dev(x), out)
            o = host(out)
            pt, lo, hi = o[E:2 * E], o[2 * E:3 * E], o[3 * E:]
            assert np.all(lo <= ref) and np.all(ref <= hi), (t, np.flatnonzero((lo > ref) | (ref > hi))[:5])
            assert np.all(lo <= pt) and np.all(pt <= hi)
            assert np.all(np.isfinite(lo)) and np.all(np.isfinite(hi))
            worst = max(worst, float(np.max(hi - lo)))
    finally:
        ctx.close()
    log(f"H={H_} scale {scale}: reference biased scores inside the bounds for 6 x {E} experts; widest {worst:.3g}")


def test_certifier_give_up_is_reported_and_recovered():
    """The certifying block's bounded wait for the rows, forced from the
    host (warp_hip_set_cert_polls: a limit of one poll, far below the rows'
    time at H 7168): a launch that gives up leaves empty job lists, so the
    layer's launches skip their work and its outputs are NaN, and the call
    reports E_DEVICE. The report resets the router's launch counter and
    tagged rows once the stream is idle: rows written after a give-up carry
    the next launch's tag, and must not pass for the next launch's rows. With
    the default limit again, picks and outputs are the oracle's."""
    import warp_amd
    E, K, H_ = 384, 8, 7168
    spec = ct.Spec(hidden=H_, inter=64, experts=E, top_k=K, layers=1, fmt="VQ12", seed=12, bias=True,
                   shared_bits=0, renorm=True, routed_scale=1.0, subnormals=False, keep_codes=False,
                   materialize=tuple(range(0, E, 8)), book_std=0.3)
    model = ct.build(spec)
    lay = model.layers[0]
    b = np.zeros(E, np.float32)
    b[::8] = 1.0                                          # the picks among the materialised experts
    lay.bias = b
    ctx = open_ctx(model)
    rng = np.random.default_rng(12)
    try:
        warp_amd.load_container_model(ctx, model)
        ctx.set_router(0, np.ascontiguousarray(lay.router, np.float32), b)
        ctx.set_cert_polls(1)
        gave_up = 0
        for t in range(4):
            x = rng.normal(size=H_).astype(np.float32)
            out = empty(H_)
            try:
                idx, _ = ctx.moe_decode(0, dev(x), out, want_route=True)
            except warp_amd.WarpHipError as e:
                assert e.code == warp_amd.E_DEVICE, e
                assert np.isnan(host(out)).all(), "a layer whose certifier gave up was computed"
                gave_up += 1
                continue
            ro, ri, _, _ = po.LayerView(model, 0).moe_layer(x)
            assert np.array_equal(idx, ri) and rel_err(host(out), ro) <= TOL
        assert gave_up >= 1, "no launch gave up after one poll"
        ctx.set_cert_polls(0)
        for t in range(4):
            x = rng.normal(size=H_).astype(np.float32)
            ro, ri, _, _ = po.LayerView(model, 0).moe_layer(x)
            out = empty(H_)
            idx, _ = ctx.moe_decode(0, dev(x), out, want_route=True)
            assert np.array_equal(idx, ri), (t, idx, ri)
            e = rel_err(host(out), ro)
            assert e <= TOL, (t, e)
    finally:
        ctx.close()
    log(f"one-poll limit: {gave_up} of 4 launches gave up (E_DEVICE, NaN layer); default limit after: picks and "
        f"outputs the oracle's on 4 tokens")
