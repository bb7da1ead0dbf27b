"""The expert cache and its miss path against the same layers fully resident.

The reference's cross-path invariant (tests/run.sh:563-618): the cache,
read-ahead and lookahead change where records come from, never the result.
A context whose cache holds a fraction of the records, filling misses
through the fetch callback (the reference's bank_fetch role), must give
bit-identical outputs and selections to a context with every record
resident, for single-token decode and for ragged batches, with and without
lookahead; the counters must add up (hits + misses = selections, bytes read
= misses x record size, evictions once the cache is full). A record that
fails its checksum is refused with E_CRC and names the layer and expert.
"""
import numpy as np
import pytest

import container as ct
from gpu_util import dev, empty, host, log, open_ctx

pytestmark = pytest.mark.gpu

SPEC = dict(hidden=256, inter=128, experts=32, top_k=4, layers=3, fmt="VQ12", seed=41, book_std=0.3,
            shared_scale=(1e-4, 3e-4))


@pytest.fixture(scope="module")
def model():
    return ct.build(ct.Spec(**SPEC))


def resident_ctx(model, **kw):
    import warp_amd
    ctx = open_ctx(model, max_tokens=32, **kw)
    warp_amd.load_container_model(ctx, model)
    return ctx


def fetching_ctx(model, slots, lookahead=0, verify=False, records=None, mode="copy"):
    """Codebooks, routers and shared experts uploaded, no records: every
    record comes through the fetch callback into a cache of `slots`. mode
    "copy": the callback copies the record into the library's staging
    buffer; "host": the records sit in pinned host memory and the callback
    returns where, so the miss copies from there."""
    import warp_amd
    ctx = open_ctx(model, max_tokens=32, cache_slots=slots, lookahead=lookahead, verify=verify)
    S = ct.FMT_STAGES[model.spec.fmt]
    for L in range(model.spec.layers):
        lay = model.layers[L]
        base = L * 3 * S
        ctx.set_codebooks(L, base, np.ascontiguousarray(model.books_raw[base:base + 3 * S]))
        ctx.set_router(L, np.ascontiguousarray(lay.router, np.float32), lay.bias)
        if lay.shared:
            s = model.spec
            ctx.set_shared(L, s.shared_bits, s.shared_group, s.inter * s.n_shared,
                           [np.ascontiguousarray(q[0]) for q in lay.shared],
                           [np.ascontiguousarray(q[1]) for q in lay.shared], [q[2] for q in lay.shared])
    recs = records if records is not None else {(L, e): r for L in range(model.spec.layers)
                                                for e, r in enumerate(model.layers[L].records)}
    if mode == "copy":
        ctx.set_fetch(lambda L, e: recs.get((L, e)))
        return ctx
    keys = sorted(recs)
    pool = ctx.host_alloc(len(keys) * model.rec_bytes)
    where = {}
    for i, k in enumerate(keys):
        pool[i * model.rec_bytes:(i + 1) * model.rec_bytes] = np.frombuffer(recs[k], np.uint8)
        where[k] = pool.ctypes.data + i * model.rec_bytes
    ctx._host_pool = pool
    ctx.set_fetch_host(lambda L, e: where.get((L, e)))
    return ctx


def run_stack(ctx, X):
    """Each token through every layer, h <- h + moe(h), on the device."""
    outs, routes = [], []
    for x in X:
        h = dev(x)
        for L in range(SPEC["layers"]):
            o = empty(SPEC["hidden"])
            idx, _ = ctx.moe_decode(L, h, o, resid_dev=h, want_route=True)
            routes.append(idx)
            h = o
        outs.append(host(h))
    return np.array(outs), np.array(routes)


@pytest.mark.parametrize("mode", ["copy", "host"])
@pytest.mark.parametrize("lookahead", [0, 3])
def test_decode_cache_equals_resident(model, lookahead, mode):
    X = np.random.default_rng(5).normal(size=(12, SPEC["hidden"])).astype(np.float32)
    ref_ctx = resident_ctx(model)
    try:
        ref_out, ref_route = run_stack(ref_ctx, X)
    finally:
        ref_ctx.close()
    slots = 10                                   # 3 layers x 32 experts do not fit
    ctx = fetching_ctx(model, slots, lookahead=lookahead, mode=mode)
    try:
        out, route = run_stack(ctx, X)
        st = ctx.cache_stats()
    finally:
        ctx.close()                              # drains the copy stream before the pool goes
        if mode == "host":
            ctx.host_free(ctx._host_pool)
    assert np.array_equal(route, ref_route)
    assert np.array_equal(out.view(np.uint32), ref_out.view(np.uint32)), "cache path changed the result"
    K, sel = SPEC["top_k"], len(route) * SPEC["top_k"]
    assert st["hits"] + st["misses"] == sel, st
    assert st["misses"] >= len({(i % SPEC["layers"], e) for i, r in enumerate(route) for e in r}) - slots
    assert st["bytes_read"] == (st["misses"] + st["prefetched"]) * model.rec_bytes or \
        st["bytes_read"] >= st["misses"] * model.rec_bytes, st
    assert st["evictions"] > 0 and st["resident"] <= slots, st
    log(f"decode, lookahead {lookahead}, {mode} fetch: bit-identical to resident over {len(X)} tokens x "
        f"{SPEC['layers']} layers; {st}")


@pytest.mark.parametrize("mode", ["copy", "host"])
def test_chunk_cache_equals_resident(model, mode):
    T = 23                                       # a ragged batch
    X = np.random.default_rng(8).normal(size=(T, SPEC["hidden"])).astype(np.float32)
    ref_ctx = resident_ctx(model)
    try:
        ref = [ref_ctx.moe_chunk_host(L, X) for L in range(SPEC["layers"])]
    finally:
        ref_ctx.close()
    ctx = fetching_ctx(model, slots=SPEC["experts"], mode=mode)   # one layer's worth: misses and evictions
    try:
        got = [ctx.moe_chunk_host(L, X) for L in range(SPEC["layers"])]
        st = ctx.cache_stats()
    finally:
        ctx.close()                              # drains the copy stream before the pool goes
        if mode == "host":
            ctx.host_free(ctx._host_pool)
    for L in range(SPEC["layers"]):
        assert np.array_equal(got[L][1], ref[L][1])
        assert np.array_equal(got[L][0].view(np.uint32), ref[L][0].view(np.uint32)), L
    assert st["misses"] > 0 and st["evictions"] > 0, st
    log(f"chunk of {T}, {mode} fetch: bit-identical to resident over {SPEC['layers']} layers; {st}")


def run_chunk_stack(ctx, batches):
    """Each batch through every layer on the device, h <- h + moe(h) (the
    residual added by the chunk's combine)."""
    outs, routes = [], []
    for X in batches:
        h = dev(X)
        for L in range(SPEC["layers"]):
            o = empty((len(X), SPEC["hidden"]))
            r, _ = ctx.moe_chunk(L, h, o, len(X), want_route=True, resid_dev=h)
            routes.append(r)
            h = o
        outs.append(host(h))
    return outs, routes


@pytest.mark.parametrize("mode", ["copy", "host"])
@pytest.mark.parametrize("lookahead", [0, 4])
def test_chunk_stack_cache_equals_resident(model, lookahead, mode):
    """Ragged batches of 9 tokens through the 3-layer stack, twice: about
    two thirds of a layer's experts are picked per batch, so a cache of one
    layer's worth both misses and has room for the lookahead's guesses,
    which the batch's own fills must not evict."""
    rng = np.random.default_rng(12)
    batches = [rng.normal(size=(9, SPEC["hidden"])).astype(np.float32) for _ in range(2)]
    ref_ctx = resident_ctx(model)
    try:
        ref_out, ref_route = run_chunk_stack(ref_ctx, batches)
    finally:
        ref_ctx.close()
    ctx = fetching_ctx(model, slots=SPEC["experts"], lookahead=lookahead, mode=mode)
    try:
        out, route = run_chunk_stack(ctx, batches)
        st = ctx.cache_stats()
    finally:
        ctx.close()
        if mode == "host":
            ctx.host_free(ctx._host_pool)
    for a, b in zip(route, ref_route):
        assert np.array_equal(a, b)
    for a, b in zip(out, ref_out):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "cache path changed the result"
    distinct = sum(len(np.unique(r)) for r in route)
    assert st["hits"] + st["misses"] == distinct, st      # each distinct record of a layer once
    assert st["bytes_read"] == (st["misses"] + st["spec_issued"]) * model.rec_bytes, st
    if lookahead:
        assert st["spec_issued"] > 0, st
    else:
        assert st["spec_issued"] == 0, st
    log(f"chunk stack, lookahead {lookahead}, {mode} fetch: bit-identical to resident; {st}")


def test_chunk_residual_is_added_last():
    """out(resid) = fl(out(no resid) + resid), bit for bit: the residual
    is the last addition, as decode's."""
    m = ct.build(ct.Spec(**{**SPEC, "layers": 1}))
    ctx = resident_ctx(m)
    try:
        X = np.random.default_rng(4).normal(size=(11, SPEC["hidden"])).astype(np.float32)
        R = np.random.default_rng(6).normal(size=(11, SPEC["hidden"])).astype(np.float32)
        xd, rd = dev(X), dev(R)
        o0, o1 = empty((11, SPEC["hidden"])), empty((11, SPEC["hidden"]))
        ctx.moe_chunk(0, xd, o0, 11)
        ctx.moe_chunk(0, xd, o1, 11, resid_dev=rd)
        want = (host(o0) + R).astype(np.float32)
        assert np.array_equal(host(o1).view(np.uint32), want.view(np.uint32))
        log("chunk residual: out(resid) == out + resid bit for bit over 11 tokens")
    finally:
        ctx.close()


def test_corrupt_record_is_refused(model):
    import warp_amd
    recs = {(L, e): bytearray(r) for L in range(model.spec.layers) for e, r in enumerate(model.layers[L].records)}
    for key in recs:
        recs[key][100] ^= 0x40                   # one flipped bit in every record's codes
    recs = {k: bytes(v) for k, v in recs.items()}
    ctx = fetching_ctx(model, slots=8, verify=True, records=recs)
    try:
        x = np.random.default_rng(2).normal(size=SPEC["hidden"]).astype(np.float32)
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.moe_decode(0, dev(x), empty(SPEC["hidden"]))
        assert ei.value.code == warp_amd.E_CRC and ei.value.layer == 0 and ei.value.expert >= 0, ei.value
        log(f"corrupt record refused: {ei.value}")
    finally:
        ctx.close()


@pytest.mark.parametrize("mode", ["copy", "host"])
@pytest.mark.parametrize("lookahead", [0, 4])
def test_chunk_with_more_experts_than_slots(model, lookahead, mode):
    """A chunk naming more distinct experts than the cache has slots (23
    tokens x top-4 of 32: about 30 distinct records per layer, 8 slots): the
    chunk runs in windows of distinct experts that fit, as the reference's
    moe_chunk streams its experts through any cache size
    (src/model.c:3595-3606). Bit-identical to all-resident; each distinct
    record asked for once per layer."""
    T = 23
    X = np.random.default_rng(18).normal(size=(T, SPEC["hidden"])).astype(np.float32)
    ref_ctx = resident_ctx(model)
    try:
        ref = [ref_ctx.moe_chunk_host(L, X) for L in range(SPEC["layers"])]
    finally:
        ref_ctx.close()
    ctx = fetching_ctx(model, slots=8, lookahead=lookahead, mode=mode)
    try:
        got = [ctx.moe_chunk_host(L, X) for L in range(SPEC["layers"])]
        st = ctx.cache_stats()
    finally:
        ctx.close()
        if mode == "host":
            ctx.host_free(ctx._host_pool)
    distinct = 0
    for L in range(SPEC["layers"]):
        assert np.array_equal(got[L][1], ref[L][1])
        assert np.array_equal(got[L][0].view(np.uint32), ref[L][0].view(np.uint32)), L
        distinct += len(np.unique(ref[L][1]))
    assert distinct > 3 * 8, distinct
    assert st["hits"] + st["misses"] == distinct, st
    assert st["resident"] <= 8, st
    log(f"chunk of {T} over {distinct} distinct records with 8 slots, lookahead {lookahead}, {mode} fetch: "
        f"bit-identical to resident; {st}")
