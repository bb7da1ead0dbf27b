"""The HIP path against the compiled reference's own outputs.

tests/golden/*.npz hold what the reference (oracle/_ref, built from its
sources) computed on the synthetic containers of tests/golden/specs.py:
moe_layer per token (output, selection, router logits), moe_chunk on 6
tokens (output, route, weights) and vq_matvec of every matrix kind of
expert 1. Here the same container bytes go through the C ABI, and each
result is compared with those stored outputs directly, not through the
oracle. The specs cover the F32, Q8G and Q4G routers (the quantised ones
through the mvq rows kernel), the SiTU activation, the VQ3R, VQ2R and
VQ4P formats, an exact router tie and a latent MoE (experts on a
projection of the hidden state, RMS norm and up projection after them).

Bars: selection and chunk routes bit-exact; strict F32 router logits
bit-exact; VQ4P matvecs bit-exact; everything else max|d|/max|ref| <= 1e-4.
"""
import os

import numpy as np
import pytest

import container as ct
from gpu_util import dev, empty, host, log, open_ctx, rel_err
from specs import SPECS

pytestmark = pytest.mark.gpu
TOL = 1e-4
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", params=sorted(SPECS))
def golden(request):
    import warp_amd
    name = request.param
    spec = SPECS[name]
    model = ct.build(spec)
    g = dict(np.load(os.path.join(HERE, f"{name}.npz")))
    assert ct.digest(model) == g["digest"].tobytes().decode(), f"{name}: container generator drifted"
    ctx = open_ctx(model, max_tokens=8)
    warp_amd.load_container_model(ctx, model)
    yield name, spec, model, g, ctx
    ctx.close()


@pytest.mark.parametrize("path", ["auto", "mfma", "gather"])
def test_moe_layer_against_reference_outputs(golden, path):
    name, spec, model, g, ctx = golden
    ctx.set_matvec_path(path)
    worst = 0.0
    try:
        for L in range(spec.layers):
            for t in range(g[f"L{L}_x"].shape[0]):
                out = empty(spec.hidden)
                idx, _ = ctx.moe_decode(L, dev(g[f"L{L}_x"][t]), out, want_route=True)
                assert np.array_equal(idx, g[f"L{L}_idx"][t]), (name, L, t, idx, g[f"L{L}_idx"][t])
                e = rel_err(host(out), g[f"L{L}_out"][t])
                worst = max(worst, e)
                assert e <= TOL, (name, path, L, t, e)
    finally:
        ctx.set_matvec_path("auto")
    log(f"[{name}] moe_layer ({path}): selections bit-exact, worst rel err {worst:.2e} against the reference")


def test_moe_chunk_against_reference_outputs(golden):
    name, spec, model, g, ctx = golden
    worst = 0.0
    for L in range(spec.layers):
        out, route, rw = ctx.moe_chunk_host(L, g[f"L{L}_chunk_x"])
        assert np.array_equal(route, g[f"L{L}_chunk_route"]), (name, L)
        ref_w = g[f"L{L}_chunk_w"]
        assert np.allclose(rw, ref_w, rtol=1e-5, atol=0), (name, L, float(np.max(np.abs(rw - ref_w))))
        e = rel_err(out, g[f"L{L}_chunk_out"])
        worst = max(worst, e)
        assert e <= TOL, (name, L, e)
    log(f"[{name}] moe_chunk: routes bit-exact, worst rel err {worst:.2e} against the reference")


def test_vq_matvec_against_reference_outputs(golden):
    name, spec, model, g, ctx = golden
    for L in range(spec.layers):
        rec = ctx.resident(L, 1)
        assert rec
        for kind in range(3):
            M = spec.inter if kind < 2 else (spec.latent or spec.hidden)
            y = empty(M)
            ctx.vq_matvec(L, kind, rec, dev(g[f"L{L}_mv{kind}_x"]), y)
            ref = g[f"L{L}_mv{kind}_y"]
            if spec.fmt == "VQ4P":
                assert np.array_equal(host(y).view(np.uint32), ref.view(np.uint32)), (name, L, kind)
            else:
                assert rel_err(host(y), ref) <= TOL, (name, L, kind, rel_err(host(y), ref))
    log(f"[{name}] vq_matvec of expert 1, every kind, within the bar against the reference")


def test_router_logits_against_reference(golden):
    """F32 routers in strict mode give the reference's logits bit for bit;
    the quantised routers (Q8G, Q4G through the mvq rows kernel) within
    the fp32 summation bound of their exact products."""
    import warp_amd
    name, spec, model, g, ctx = golden
    if spec.router == "f32":
        sctx = open_ctx(model, max_tokens=8, router_strict=True)
        try:
            warp_amd.load_container_model(sctx, model)
            for L in range(spec.layers):
                X = g[f"L{L}_x"]
                lg = empty((X.shape[0], spec.experts))
                sctx.router_logits(L, dev(X), X.shape[0], lg)
                assert np.array_equal(host(lg).view(np.uint32), g[f"L{L}_logits"].view(np.uint32)), (name, L)
        finally:
            sctx.close()
        log(f"[{name}] strict F32 router logits bit-exact against the reference")
        return
    for L in range(spec.layers):
        X = g[f"L{L}_x"]
        lg = empty((X.shape[0], spec.experts))
        ctx.router_logits(L, dev(X), X.shape[0], lg)
        W = dequant_rows(*model.layers[L].router_q, spec.hidden)
        ref = g[f"L{L}_logits"].astype(np.float64)
        # both sums round each of at most H additions: |d| <= 2 H u sum|w x|
        bound = 2 * spec.hidden * 2.0 ** -24 * (np.abs(X).astype(np.float64) @ np.abs(W).T)
        d = np.abs(host(lg) - ref)
        assert np.all(d <= bound), (name, L, float(np.max(d / bound)))
        exact = X.astype(np.float64) @ W.T
        assert np.all(np.abs(ref - exact) <= bound), "the dequantisation here does not match the reference's"
    log(f"[{name}] Q{spec.router[1:]}G router logits within the fp32 bound of the reference's")


def dequant_rows(payload, scales, rowbytes, bits, group, N):
    """Q8G / Q4G rows (int8, or two 4-bit values + 8 per byte, low nibble
    first) times their fp16 group scales, in float64."""
    p = np.asarray(payload, np.uint8)
    if bits == 8:
        q = p.view(np.int8).astype(np.float64)
    else:
        q = np.empty((p.shape[0], 2 * p.shape[1]))
        q[:, 0::2] = (p & 15).astype(np.float64) - 8
        q[:, 1::2] = (p >> 4).astype(np.float64) - 8
    s = np.asarray(scales, np.uint16).view(np.float16).astype(np.float64)
    return (q * np.repeat(s, group, axis=1)[:, :q.shape[1]])[:, :N]
