"""The latent MoE (src/model.c:2898-2939) on the GPU against the oracle: the
experts run on x_lat = routed_expert_down_proj . x, their weighted sum is
RMS-normalised (latent_moe_use_norm), projected back up with
routed_expert_up_proj, and the shared expert and the residual are added;
routing stays on x. Hidden 1024, latent 512, inter 256, 64 experts, top-6,
Q8G g32 projections and shared expert; VQ3R and VQ4P records.

- decode on every matvec path (the table kernel, the decode-then-dot kernel;
  VQ4P's int8-table kernel), selections bit-exact, outputs within the bar;
- the chunk on 16 tokens, with a cache that holds every expert and with one
  that holds 8 slots (the chunk's experts then stream through it in windows);
- the vector expert FFN on latent-width inputs;
- a context with a latent width but a layer without its projections refuses
  the layer instead of running the experts on the wrong width.
"""
import numpy as np
import pytest

import container as ct
from gpu_util import dev, empty, host, log, open_ctx, rel_err
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4
SHAPE = dict(hidden=1024, inter=256, experts=64, top_k=6, layers=1, latent=512, shared_bits=8, shared_group=32,
             subnormals=False, keep_codes=False, routed_scale=2.5, bias=True, renorm=True)


def model_of(fmt, norm=True):
    return ct.build(ct.Spec(fmt=fmt, router="f32", latent_norm=norm, seed=61 + (fmt == "VQ4P"), **SHAPE))


@pytest.mark.parametrize("fmt,norm", [("VQ3R", True), ("VQ4P", True), ("VQ3R", False)])
def test_latent_decode(fmt, norm):
    import warp_amd
    model = model_of(fmt, norm)
    ctx = open_ctx(model)
    ref = po.LayerView(model, 0)
    try:
        warp_amd.load_container_model(ctx, model)
        rng = np.random.default_rng(5)
        worst = {}
        for path in ("auto", "mfma", "gather"):
            ctx.set_matvec_path(path)
            w = 0.0
            for t in range(6):
                x = rng.normal(size=SHAPE["hidden"]).astype(np.float32)
                yr, ir, _, _ = ref.moe_layer(x)
                out = empty(SHAPE["hidden"])
                idx, _ = ctx.moe_decode(0, dev(x), out, want_route=True)
                assert np.array_equal(idx, ir), (path, t, idx, ir)
                e = rel_err(host(out), yr)
                w = max(w, e)
                assert e <= TOL, (fmt, path, t, e)
            worst[path] = w
        ctx.set_matvec_path("auto")
        log(f"latent decode {fmt} norm={norm}: selections bit-exact, worst rel err " +
            ", ".join(f"{p} {v:.2e}" for p, v in worst.items()))
    finally:
        ctx.close()


@pytest.mark.parametrize("slots", [None, 8])
def test_latent_chunk(slots):
    import warp_amd
    model = model_of("VQ3R")
    ctx = open_ctx(model, max_tokens=16, cache_slots=slots)
    ref = po.LayerView(model, 0)
    try:
        if slots is None:
            warp_amd.load_container_model(ctx, model)
        else:
            # records come through the fetch function, a window at a time
            warp_amd.load_container_model(ctx, model, records=False)
            recs = model.layers[0].records
            ctx.set_fetch(lambda L, e: recs[e])
        X = np.random.default_rng(9).normal(size=(16, SHAPE["hidden"])).astype(np.float32)
        yr, rr, wr = ref.moe_chunk(X)
        out, route, rw = ctx.moe_chunk_host(0, X)
        assert np.array_equal(route, rr)
        assert np.allclose(rw, wr, rtol=1e-6, atol=0)
        e = rel_err(out, yr)
        assert e <= TOL, e
        n = len(np.unique(rr))
        assert slots is None or n > slots
        log(f"latent chunk, 16 tokens, {n} distinct experts, slots {slots or 'all'}: routes bit-exact, "
            f"rel err {e:.2e}")
    finally:
        ctx.close()


def test_latent_expert_ffn():
    import warp_amd
    model = model_of("VQ3R")
    ctx = open_ctx(model)
    try:
        warp_amd.load_container_model(ctx, model)
        lat = SHAPE["latent"]
        x = np.random.default_rng(3).normal(size=lat).astype(np.float32)
        bT = po.books_T(model.books_raw)
        rec = np.frombuffer(model.layers[0].records[7], np.uint8)
        hdr = np.frombuffer(model.layers[0].records[7][:48], np.uint32)
        S = ct.FMT_STAGES["VQ3R"]
        I = SHAPE["inter"]
        corr = int(hdr[8])

        def mat(kind):
            M, N = (I, lat) if kind < 2 else (lat, I)
            soff = [0, I, 2 * I][kind]
            return (rec[int(hdr[5 + kind]):].copy(), rec[corr + 2 * soff: corr + 2 * (soff + M)].view(np.uint16).copy(),
                    M, N)

        g = po.vq_matvec("VQ3R", *mat(0)[:2], x, bT, 0, I, lat)
        u = po.vq_matvec("VQ3R", *mat(1)[:2], x, bT, S, I, lat)
        h = (np.array([po.lib().or_silu(float(v)) for v in g], np.float32) * u).astype(np.float32)
        yr = po.vq_matvec("VQ3R", *mat(2)[:2], h, bT, 2 * S, lat, I)
        for path in ("auto", "mfma", "gather"):
            ctx.set_matvec_path(path)
            y = empty(lat)
            ctx.expert_ffn(0, 7, dev(x), y)
            ctx.sync()
            e = rel_err(host(y), yr)
            assert e <= TOL, (path, e)
        ctx.set_matvec_path("auto")
        log("latent expert FFN (512 wide) within the bar on both kernels")
    finally:
        ctx.close()


def test_latent_layer_without_projections_refused():
    import warp_amd
    model = model_of("VQ3R")
    ctx = open_ctx(model)
    try:
        lay = model.layers[0]
        saved, lay.latent = lay.latent, None
        try:
            warp_amd.load_container_model(ctx, model)
        finally:
            lay.latent = saved
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.moe_decode(0, dev(np.zeros(SHAPE["hidden"], np.float32)), empty(SHAPE["hidden"]))
        assert ei.value.code == warp_amd.E_ARG
        log("latent layer without projections refused with E_ARG")
    finally:
        ctx.close()
