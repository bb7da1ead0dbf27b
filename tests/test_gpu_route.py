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
