"""A decode step captured into a HIP graph and replayed.

With every record resident (or no fetch function), warp_hip_moe_decode
issues only kernels and event records on the context's stream, so a caller
can capture a step of several layers into a graph and replay it per token.
Each replay must equal the same step launched from the host, bit for bit,
also with eager work and synchronisations of the same context between the
replays: the K3-shape path (routing inside the gate/up launch, no shared
expert) and a layer with a Q8G shared expert (inside the router and combine
launches).

The same for a stack of chunks: with every record resident and no routes
asked for, warp_hip_moe_chunk queues its work (the shared expert on a side
stream joined back by events) and returns, so a step can be captured too.
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


@pytest.mark.parametrize("fp16", [False, True])
def test_chunk_graph_replays_equal_eager(fp16):
    """A 2-layer stack of chunks (every record resident, no routes asked
    for, so a chunk queues its work and returns; a Q8G shared expert on its
    side stream) captured into a graph and replayed 4 times, with eager
    chunks and synchronisations between the replays: every replay's outputs
    equal the eager step's bit for bit, in both precision modes."""
    import warp_amd
    from warp_amd.device import D2D, Graph, copy_async
    spec = ct.Spec(hidden=512, inter=256, experts=32, top_k=4, layers=2, fmt="VQ12", seed=37, shared_bits=8,
                   **BALANCED)
    model = ct.build(spec)
    T = 24
    ctx = open_ctx(model, max_tokens=T, prefill_fp16=fp16)
    try:
        warp_amd.load_container_model(ctx, model)
        H, Lyr = spec.hidden, spec.layers
        rng = np.random.default_rng(41)
        Xs = [dev(rng.normal(size=(T, H)).astype(np.float32)) for _ in range(4)]
        stage = empty((T, H))
        outs = [empty((T, H)) for _ in range(Lyr)]

        def step(x_ptr):
            for L in range(Lyr):
                ctx.moe_chunk(L, x_ptr if L == 0 else outs[L - 1].ptr, outs[L].ptr, T)

        # eager references
        ref = []
        for x in Xs:
            step(x.ptr)
            ctx.sync()
            ref.append([host(o).copy() for o in outs])
        g = Graph(ctx.stream, lambda: step(stage.ptr))
        try:
            for rep in range(4):
                ctx.moe_chunk(0, Xs[(rep + 1) % 4].ptr, empty((T, H)).ptr, T)      # eager work between replays
                ctx.sync()
                copy_async(stage.ptr, Xs[rep].ptr, T * H * 4, D2D, ctx.stream)
                g.launch()
                ctx.sync()
                for L in range(Lyr):
                    assert np.array_equal(host(outs[L]).view(np.uint32), ref[rep][L].view(np.uint32)), (rep, L)
        finally:
            g.free()
        log(f"chunk stack (prefill_fp16={fp16}): 4 graph replays bit-identical to the eager steps")
    finally:
        ctx.close()
