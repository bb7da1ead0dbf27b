"""The HBM expert cache's accounting against the reference's expert cache on
the reference's own routing trace.

tests/golden/trace_kimi_300.npz holds the reference's real Kimi-Linear
routing (its tests/trace_kimi_300.jsonl: 300 tokens x 26 MoE layers x top-8
of 256) and what its cache (src/ecache.c, compiled from its sources)
counted replaying it with read-ahead and lookahead off, at several cache
sizes. Here the same selections go through warp_hip_moe_decode on a small
container (router weights zero, the bias ordering each token's eight ids
first) with a cache of the same number of slots, misses filled through the
fetch function. The victim choice is the reference's (lowest empty slot,
then LFRU over 16 slots sampled with its generator); the one difference is
that a decode holds its whole selection while the reference holds only the
record in use, so the counters are compared the way the reference compares
its trace simulator with its engine (tests/run.sh:584-606): hit rates
within 5 points. Hits plus misses equal the records asked for, exactly.
"""
import os
import struct

import numpy as np
import pytest

import container as ct
from gpu_util import dev, empty, log, open_ctx

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("slots", [208, 1024])
def test_hit_rate_follows_the_reference_cache(slots):
    g = dict(np.load(os.path.join(HERE, "trace_kimi_300.npz")))
    ids = g["ids"].astype(np.int64)
    n_tok, n_layers, K = ids.shape
    ref = g["ref_counts"][list(g["slots"]).index(slots)]
    spec = ct.Spec(hidden=64, inter=32, experts=256, top_k=K, layers=1, fmt="VQ3R", seed=23, bias=True,
                   shared_bits=0, subnormals=False, keep_codes=False, materialize=(0,), renorm=False)
    one = ct.build(spec)
    template = bytearray(one.layers[0].records[0])

    def fetch(L, e):
        r = bytearray(template)
        struct.pack_into("<HH", r, 4, L, e)                 # the header names the record asked for
        return bytes(r)
    big = ct.Spec(**{**spec.__dict__, "layers": n_layers})
    model = ct.Model(spec=big, books_raw=np.zeros((n_layers * 9, 256, 8), np.uint16), layers=[], rec_bytes=one.rec_bytes)
    ctx = open_ctx(model, max_tokens=1, cache_slots=slots)
    try:
        zeros = np.zeros((256, 64), np.float32)
        for L in range(n_layers):
            ctx.set_codebooks(L, L * 9, np.zeros((9, 256, 8), np.uint16))
        ctx.set_fetch(fetch)
        x = dev(np.zeros(64, np.float32))
        out = empty(64)
        bias = np.zeros(256, np.float32)
        for t in range(n_tok):
            for L in range(n_layers):
                bias[:] = 0.0
                bias[ids[t, L]] = 1.0 - 0.01 * np.arange(K, dtype=np.float32)
                ctx.set_router(L, zeros, bias)
                idx, _ = ctx.moe_decode(L, x, out, want_route=True)
                assert np.array_equal(idx, ids[t, L]), (t, L)
        st = ctx.cache_stats()
    finally:
        ctx.close()
    asked = n_tok * n_layers * K
    assert st["hits"] + st["misses"] == asked == int(ref[0] + ref[1])
    ours, theirs = st["hits"] / asked, float(ref[0]) / asked
    assert abs(ours - theirs) <= 0.05, (ours, theirs)
    log(f"trace replay, {slots} slots: hit rate {ours:.4f} here, {theirs:.4f} in the reference's cache "
        f"(hits {st['hits']} vs {int(ref[0])}, evictions {st['evictions']} vs {int(ref[2])})")
