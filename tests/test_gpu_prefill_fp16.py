"""A chunk's reduced-precision mode (prefill_fp16: each position's stage
vectors added into one fp16 value, x's fp16 high half only, SwiGLU's SiLU
with the hardware exp, products accumulated in fp32 on the matrix cores)
against the reference's outputs
and the oracle, through the C ABI.

The bar for this mode is max|d|/max|ref| <= 2e-3, ten times inside the
2e-2 that a bf16-operand prefill is allowed; routes and weights stay
bit-exact (routing does not go through the expert products). A token sent
to the wrong B column or a dropped stage moves the output by O(1), far
outside the bar.

- the reference's stored chunk outputs (tests/golden, VQ3R, VQ2R, SiTU,
  router ties, latent MoE);
- the Kimi-Linear prefill shape on 64 tokens against the oracle's
  moe_chunk, both routings, Zipf-skewed runs (odd and even job counts);
- 512 tokens: token order changes no result bit, and every token stays
  within the bar of the exact mode's chunk output;
- chunks of 1, 3 and 9 tokens (runs of a single partial job);
- rows that do not fill 64-row blocks (hidden 160, intermediate 96), both
  modes;
- more distinct experts than cache slots (windows), bit-identical to a
  cache that holds them all.
"""
import os

import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, log, open_ctx, rel_err
from oracle import pyoracle as po
from specs import SPECS
from test_gpu_configs import ACTS, KIMI, zipf_model

pytestmark = pytest.mark.gpu
TOL16 = 2e-3
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name", sorted(n for n in SPECS if SPECS[n].fmt != "VQ4P"))
def test_fp16_chunk_against_reference_outputs(name):
    import warp_amd
    spec = SPECS[name]
    model = ct.build(spec)
    g = dict(np.load(os.path.join(HERE, f"{name}.npz")))
    assert ct.digest(model) == g["digest"].tobytes().decode(), f"{name}: container generator drifted"
    ctx = open_ctx(model, max_tokens=8, prefill_fp16=True)
    try:
        warp_amd.load_container_model(ctx, model)
        worst = 0.0
        for L in range(spec.layers):
            out, route, rw = ctx.moe_chunk_host(L, g[f"L{L}_chunk_x"])
            assert np.array_equal(route, g[f"L{L}_chunk_route"]), (name, L)
            assert np.allclose(rw, g[f"L{L}_chunk_w"], rtol=1e-5, atol=0), (name, L)
            e = rel_err(out, g[f"L{L}_chunk_out"])
            worst = max(worst, e)
            assert e <= TOL16, (name, L, e)
        log(f"[{name}] fp16 chunk: routes bit-exact, worst rel err {worst:.2e} against the reference")
    finally:
        ctx.close()


@pytest.mark.parametrize("act", sorted(ACTS))
def test_fp16_config3_prefill_64_against_oracle(act):
    import warp_amd
    model, _ = zipf_model("VQ12", 4, act=act)
    ctx = open_ctx(model, max_tokens=64, cache_slots=48, router_act=ACTS[act], prefill_fp16=True)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(5).normal(size=(64, KIMI["hidden"])).astype(np.float32)
        out, route, rw = ctx.moe_chunk_host(0, X)
        ro, rr, rrw = po.LayerView(model, 0, router_act=ACTS[act]).moe_chunk(X)
        assert np.array_equal(route, rr)
        assert np.allclose(rw, rrw, rtol=1e-5, atol=0)
        e = rel_err(out, ro)
        assert e <= TOL16, e
        counts = np.bincount(route.ravel(), minlength=256)
        jobs = (counts[counts > 0] + 7) // 8
        assert (jobs % 2 == 1).any() and (jobs > 1).any(), "runs did not cover odd and multi-job counts"
        log(f"fp16 config 3 ({act}), 64 tokens: rel err {e:.2e} against the oracle; busiest experts "
            f"{sorted(counts)[-5:]}")
    finally:
        ctx.close()


@pytest.mark.parametrize("act", sorted(ACTS))
def test_fp16_config3_prefill_512_properties(act):
    import warp_amd
    model, _ = zipf_model("VQ12", 6, act=act)
    T = 512
    X = np.random.default_rng(7).normal(size=(T, KIMI["hidden"])).astype(np.float32)
    res = {}
    for fp16 in (False, True):
        ctx = open_ctx(model, max_tokens=T, cache_slots=48, router_act=ACTS[act], prefill_fp16=fp16)
        try:
            warp_amd.load_container_model(ctx, model)
            res[fp16] = ctx.moe_chunk_host(0, X)
            if fp16:
                perm = np.random.default_rng(8).permutation(T)
                out_p, route_p, _ = ctx.moe_chunk_host(0, X[perm])
                assert np.array_equal(route_p, res[fp16][1][perm])
                assert np.array_equal(out_p.view(np.uint32), res[fp16][0][perm].view(np.uint32)), \
                    "token order changed a result"
        finally:
            ctx.close()
    assert np.array_equal(res[True][1], res[False][1])
    worst = max(rel_err(res[True][0][t], res[False][0][t]) for t in range(T))
    assert worst <= TOL16, worst
    log(f"fp16 config 3 ({act}), 512 tokens: order-invariant bit for bit, worst per-token rel err {worst:.2e} "
        f"against the exact mode")


@pytest.mark.parametrize("T", [1, 3, 9])
def test_fp16_small_chunks(T):
    import warp_amd
    spec = ct.Spec(hidden=1024, inter=512, experts=16, top_k=4, layers=1, fmt="VQ3R", seed=23, subnormals=False,
                   keep_codes=False, **BALANCED)
    model = ct.build(spec)
    ctx = open_ctx(model, max_tokens=T, prefill_fp16=True)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(T).normal(size=(T, spec.hidden)).astype(np.float32)
        out, route, _ = ctx.moe_chunk_host(0, X)
        ro, rr, _ = po.LayerView(model, 0).moe_chunk(X)
        assert np.array_equal(route, rr)
        e = rel_err(out, ro)
        assert e <= TOL16, (T, e)
        log(f"fp16 chunk of {T} tokens: rel err {e:.2e}")
    finally:
        ctx.close()


@pytest.mark.parametrize("fp16", [True, False])
def test_chunk_rows_not_a_multiple_of_64(fp16):
    """Hidden 160 and intermediate 96: neither launch's rows fill whole
    64-row blocks, so the run kernels store their outputs one row at a time
    instead of as transposed 64-byte sectors; both modes against the oracle
    (2e-3 reduced precision, 1e-4 exact)."""
    import warp_amd
    spec = ct.Spec(hidden=160, inter=96, experts=16, top_k=4, layers=1, fmt="VQ12", seed=29, subnormals=False,
                   keep_codes=False, **BALANCED)
    model = ct.build(spec)
    T = 40
    ctx = open_ctx(model, max_tokens=T, prefill_fp16=fp16)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(29).normal(size=(T, spec.hidden)).astype(np.float32)
        out, route, _ = ctx.moe_chunk_host(0, X)
        ro, rr, _ = po.LayerView(model, 0).moe_chunk(X)
        assert np.array_equal(route, rr)
        e = rel_err(out, ro)
        assert e <= (TOL16 if fp16 else 1e-4), (fp16, e)
        log(f"chunk of {T} tokens at hidden 160 / inter 96 ({'fp16' if fp16 else 'exact'}): rel err {e:.2e}")
    finally:
        ctx.close()


def test_fp16_chunk_in_windows():
    """More distinct experts than cache slots: the chunk's experts stream
    through the cache in windows (x is split per pair in the first window
    only); outputs bit-identical to a cache that holds every expert, and
    within the bar of the oracle."""
    import warp_amd
    spec = ct.Spec(hidden=1024, inter=512, experts=32, top_k=4, layers=1, fmt="VQ12", seed=31, subnormals=False,
                   keep_codes=False, **BALANCED)
    model = ct.build(spec)
    X = np.random.default_rng(17).normal(size=(24, spec.hidden)).astype(np.float32)
    outs = {}
    for slots in (None, 8):
        ctx = open_ctx(model, max_tokens=24, cache_slots=slots, prefill_fp16=True)
        try:
            if slots is None:
                warp_amd.load_container_model(ctx, model)
            else:
                warp_amd.load_container_model(ctx, model, records=False)
                recs = model.layers[0].records
                ctx.set_fetch(lambda L, e: recs[e])
            outs[slots] = ctx.moe_chunk_host(0, X)
        finally:
            ctx.close()
    (o1, r1, w1), (o2, r2, w2) = outs[None], outs[8]
    n = len(np.unique(r1))
    assert n > 8, n
    assert np.array_equal(r1, r2) and np.array_equal(w1.view(np.uint32), w2.view(np.uint32))
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32)), float(np.max(np.abs(o1 - o2)))
    ro, rr, _ = po.LayerView(model, 0).moe_chunk(X)
    assert np.array_equal(r1, rr)
    e = rel_err(o1, ro)
    assert e <= TOL16, e
    log(f"fp16 chunk of 24 over {n} distinct experts in windows of 8: bit-identical to all resident, rel err {e:.2e}")
