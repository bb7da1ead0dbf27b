"""A decode step captured into a HIP graph and replayed.

With every record resident (or no fetch function), warp_hip_moe_decode
issues only kernels and event records on the context's stream, so a caller
can capture a step of several layers into a graph and replay it per token.
Each replay must equal the same step launched from the host, bit for bit,
also with eager work and synchronisations of the same context between the
replays: the K3-shape path (routing inside the gate/up launch, no shared
expert) and a layer with a Q8G shared expert (inside the router and combine
launches).
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shared", [0, 8])
def test_decode_graph_replays_equal_eager(shared):
    import warp_amd
    from warp_amd.device import D2D, Graph, copy_async
    spec = ct.Spec(hidden=256, inter=128, experts=32, top_k=4, layers=3, fmt="VQ12", seed=29,
                   shared_bits=shared, **BALANCED)
    model = ct.build(spec)
    ctx = open_ctx(model)
    try:
        warp_amd.load_container_model(ctx, model)
        H, Lyr = spec.hidden, spec.layers
        X = np.random.default_rng(31).normal(size=(4, H)).astype(np.float32)
        xs = [dev(x) for x in X]
        stage = empty(H)
        bufs = [empty(H), empty(H)]

        def step(x_ptr):
            x = x_ptr
            for L in range(Lyr):
                out = bufs[L & 1]
                ctx.moe_decode(L, x, out, resid_dev=x)
                x = out.ptr

        eager = []
        for b in xs:
            step(b.ptr)
            eager.append(host(bufs[(Lyr - 1) & 1]).copy())
        g = Graph(ctx.stream, lambda: step(stage.ptr))
        try:
            for rep in range(3):
                for i, b in enumerate(xs):
                    copy_async(stage.ptr, b.ptr, H * 4, D2D, ctx.stream)
                    g.launch()
                    ctx.sync()
                    got = host(bufs[(Lyr - 1) & 1])
                    assert np.array_equal(got.view(np.uint32), eager[i].view(np.uint32)), (rep, i)
                    # eager work of the same context between replays
                    o = empty(H)
                    ctx.moe_decode(0, xs[(i + 1) % 4], o)
                    ctx.sync()
        finally:
            g.free()
        log(f"decode graph ({'Q8G shared expert' if shared else 'no shared expert'}): 12 replays of a "
            f"{Lyr}-layer step equal eager bit for bit")
    finally:
        ctx.close()
