"""The K3-scale miss configuration at its shape: hidden 7168, 384 experts of
intermediate 2048, top-16, 2x4096 12-bit codes, a 32-token decode batch
(one token per sequence) through a 2-layer stack, h <- h + moe(h).

Each layer has 48 expert records and its bias lifts them, so the batch's
512 picks spread over about all 48. The HBM cache holds 40 records: under
half of the stack's 96, and fewer than one layer's distinct experts, so
every layer both misses and runs in two windows of experts
(src/model.c:3595-3606 streams a chunk's experts through any cache size).
Misses are copied from pinned host memory (the set_fetch_host tier), with
lookahead 0 and 4. Against the same stack all resident: routes bit-exact
and outputs bit-identical; hits + misses = the distinct records of each
layer (src/ecache.c:596-669 counts per record asked). The resident stack's
first layer against the oracle's moe_chunk on 4 of the tokens: routes
bit-exact, output within 1e-4.
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4
H, I, E, K, LAYERS, T, N_REC, SLOTS = 7168, 2048, 384, 16, 2, 32, 48, 40


@pytest.fixture(scope="module")
def k3_stack():
    ids = tuple(int(i) for i in np.random.default_rng(5).permutation(E)[:N_REC])
    spec = ct.Spec(hidden=H, inter=I, experts=E, top_k=K, layers=LAYERS, fmt="VQ12", seed=81, shared_bits=0,
                   materialize=ids, subnormals=False, keep_codes=False, **BALANCED)
    model = ct.build(spec)
    for L in range(LAYERS):
        b = np.zeros(E, np.float32)
        b[list(ids)] = 1.0
        model.layers[L].bias = b
    X = np.random.default_rng(6).normal(size=(T, H)).astype(np.float32)
    log(f"config 5 stack built: {LAYERS} layers x {N_REC} records of {model.rec_bytes} bytes")
    return model, X


def load_weights(ctx, model):
    S = ct.FMT_STAGES[model.spec.fmt]
    for L in range(LAYERS):
        base = L * 3 * S
        ctx.set_codebooks(L, base, np.ascontiguousarray(model.books_raw[base:base + 3 * S]))
        ctx.set_router(L, np.ascontiguousarray(model.layers[L].router, np.float32), model.layers[L].bias)


def run(ctx, X):
    h = dev(X)
    outs, routes = [], []
    for L in range(LAYERS):
        o = empty((T, H))
        r, _ = ctx.moe_chunk(L, h, o, T, want_route=True, resid_dev=h)
        routes.append(r)
        outs.append(host(o))
        h = o
    return outs, routes


@pytest.fixture(scope="module")
def resident(k3_stack):
    import warp_amd
    model, X = k3_stack
    ctx = open_ctx(model, max_tokens=T, cache_slots=LAYERS * N_REC)
    try:
        warp_amd.load_container_model(ctx, model)
        outs, routes = run(ctx, X)
    finally:
        ctx.close()
    return outs, routes


def test_config5_resident_against_oracle(k3_stack, resident):
    model, X = k3_stack
    outs, routes = resident
    ro, rr, _ = po.LayerView(model, 0).moe_chunk(X[:4])
    assert np.array_equal(routes[0][:4], rr)
    # the stack adds the residual in the combine: layer 0's output is h + moe(h)
    e = rel_err(outs[0][:4] - X[:4], ro)
    assert e <= TOL, e
    log(f"config 5, resident: 4 tokens of the 32-token batch against the oracle's moe_chunk, rel err {e:.2e}; "
        f"{len(np.unique(routes[0]))} distinct experts in layer 0")


@pytest.mark.parametrize("lookahead", [0, 4])
def test_config5_half_missing_equals_resident(k3_stack, resident, lookahead):
    model, X = k3_stack
    ref_outs, ref_routes = resident
    ctx = open_ctx(model, max_tokens=T, cache_slots=SLOTS, lookahead=lookahead)
    recs = {(L, e): r for L in range(LAYERS) for e, r in enumerate(model.layers[L].records) if r is not None}
    keys = sorted(recs)
    pool = ctx.host_alloc(len(keys) * model.rec_bytes)
    try:
        load_weights(ctx, model)
        where = {}
        for i, k in enumerate(keys):
            pool[i * model.rec_bytes:(i + 1) * model.rec_bytes] = np.frombuffer(recs[k], np.uint8)
            where[k] = pool.ctypes.data + i * model.rec_bytes
        ctx.set_fetch_host(lambda L, e: where.get((L, e)))
        outs, routes = run(ctx, X)
        st = ctx.cache_stats()
    finally:
        ctx.close()                              # drains the copy stream before the pool goes
        ctx.host_free(pool)
    distinct = 0
    for L in range(LAYERS):
        assert np.array_equal(routes[L], ref_routes[L]), L
        assert np.array_equal(outs[L].view(np.uint32), ref_outs[L].view(np.uint32)), f"layer {L} changed"
        distinct += len(np.unique(ref_routes[L]))
    assert distinct > SLOTS * 2, distinct
    assert st["hits"] + st["misses"] == distinct, st
    assert st["misses"] >= distinct - SLOTS, st
    assert st["bytes_read"] == (st["misses"] + st["spec_issued"]) * model.rec_bytes, st
    log(f"config 5, {SLOTS} slots for {distinct} distinct records, lookahead {lookahead}: bit-identical to "
        f"resident; miss rate {st['misses'] / distinct:.2f}; {st}")
