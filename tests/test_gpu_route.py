"""Routing on the GPU against the oracle's restatement of the reference's
scan (src/model.c:2723-2745), on logits and biases built to tie: selection
order and weights bit-exact, for the one-token decode kernel and the
multi-token kernel, sigmoid and softmax scoring."""
import numpy as np
import pytest

from gpu_util import dev, empty, host, log
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
E, K, H = 96, 12, 64


def make_ctx(act):
    import warp_amd
    return warp_amd.Context(hidden=H, inter=32, n_experts=E, top_k=K, n_layers=1, fmt="VQ12", renorm=True,
                            routed_scale=2.5, router_act=act, max_tokens=8, rec_bytes=8192, cache_bytes=8192)


def cases(rng):
    out = []
    # equal logits in coarse steps, no bias: many exact ties of the score
    out.append((np.round(rng.normal(size=E) * 2) * 0.5, None))
    # ties of score + bias
    out.append((np.zeros(E), np.floor(rng.uniform(0, 4, E)) * 0.25))
    # a band of experts pushed to -1e30 (never picked) and exact duplicates
    lg = rng.normal(size=E)
    lg[10:20] = lg[0]
    b = np.zeros(E)
    b[40:60] = -1e30
    out.append((lg, b))
    # all equal: the lowest ids in order
    out.append((np.full(E, 0.3), np.zeros(E)))
    # distinct values except for one value shared by the 9th..15th largest,
    # so the cut at K falls inside a run of ties and only its lowest ids go
    lg = rng.normal(size=E)
    order = np.argsort(-lg, kind="stable")
    lg[order[8:15]] = lg[order[8]]
    out.append((lg, None))
    return [(np.asarray(l, np.float32), None if b is None else np.asarray(b, np.float32)) for l, b in out]


@pytest.mark.parametrize("act", [0, 1])
def test_route_ties(act):
    rng = np.random.default_rng(31 + act)
    ctx = make_ctx(act)
    try:
        router = np.zeros((E, H), np.float32)
        for n, (lg, b) in enumerate(cases(rng)):
            ctx.set_router(0, router, b)
            ri, rw, _ = po.route(lg, b, K, act, 1, 2.5)
            # one token: the decode kernel
            idx, w = empty(K, np.int32), empty(K)
            ctx.route(0, dev(lg), 1, idx, w)
            assert np.array_equal(host(idx), ri), (n, host(idx), ri)
            assert np.array_equal(host(w).view(np.uint32), rw.view(np.uint32)), (n, host(w), rw)
            # several tokens: the batched kernel, each row the same case
            T = 5
            idx5, w5 = empty((T, K), np.int32), empty((T, K))
            ctx.route(0, dev(np.tile(lg, (T, 1))), T, idx5, w5)
            for t in range(T):
                assert np.array_equal(host(idx5)[t], ri), (n, t)
                assert np.array_equal(host(w5)[t].view(np.uint32), rw.view(np.uint32)), (n, t)
        log(f"route act={act}: {len(cases(rng))} tie cases bit-exact on both kernels")
    finally:
        ctx.close()


@pytest.mark.parametrize("act", [0, 1])
def test_scores_bitexact_on_many_logits(act):
    """Every expert picked (K = E = 64, no renormalisation, scale 1), so the
    weights are the scores themselves: sigmoid 1/(1+expf(-l)) or softmax
    expf(l - max)/sum. 4096 tokens through the batched kernel and 64 through
    the one-token kernel, against the oracle (glibc's expf): selection and
    weights bit-exact. The exp arguments span the range where the score
    depends on every bit of expf, and the sample includes arguments on which
    a correctly rounded exp differs from glibc's, so only an expf that
    reproduces glibc's passes."""
    import warp_amd
    Ek, T = 64, 4096
    ctx = warp_amd.Context(hidden=64, inter=32, n_experts=Ek, top_k=Ek, n_layers=1, fmt="VQ12", renorm=False,
                           routed_scale=1.0, router_act=act, max_tokens=T, rec_bytes=8192, cache_bytes=8192)
    try:
        ctx.set_router(0, np.zeros((Ek, 64), np.float32), None)
        rng = np.random.default_rng(71 + act)
        if act == 0:
            lg = -rng.uniform(-17.0, 88.0, (T, Ek)).astype(np.float32)
            args = -lg
        else:
            lg = rng.uniform(-87.0, 0.0, (T, Ek)).astype(np.float32)
            args = lg - lg.max(axis=1, keepdims=True)
        gl = np.empty_like(args)
        po.lib().or_expf_array(args.ctypes.data, gl.ctypes.data, args.size)
        cr = np.exp(args.astype(np.float64)).astype(np.float32)
        differ = int(np.count_nonzero(gl.view(np.uint32) != cr.view(np.uint32)))
        assert differ > 0
        idx, w = empty((T, Ek), np.int32), empty((T, Ek))
        ctx.route(0, dev(lg), T, idx, w)
        gi, gw = host(idx), host(w)
        for t in range(T):
            ri, rw, _ = po.route(lg[t], None, Ek, act, 0, 1.0)
            assert np.array_equal(gi[t], ri), t
            assert np.array_equal(gw[t].view(np.uint32), rw.view(np.uint32)), t
        for t in range(64):
            i1, w1 = empty(Ek, np.int32), empty(Ek)
            ctx.route(0, dev(lg[t]), 1, i1, w1)
            assert np.array_equal(host(i1), gi[t]) and np.array_equal(host(w1).view(np.uint32), gw[t].view(np.uint32))
        log(f"route act={act}: {T * Ek} scores bit-exact with glibc's expf ({differ} arguments where a "
            f"correctly rounded exp differs)")
    finally:
        ctx.close()
