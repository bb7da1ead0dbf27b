"""Codebooks holding exponent-31 fp16 values, which the reference reads as
finite powers of two (src/simd.h:49-67; the oracle's conversion is pinned
in test_oracle_math.py), on every entry point against the oracle: decode
with the matrix-core path requested, the chunk in both precision modes,
the single-expert FFN and vq_matvec. Such a layer takes the table kernel
(its exact conversion) everywhere; the fp16 matrix-core operands would read
those values as inf/NaN. Bars as elsewhere: selections and routes
bit-exact, outputs max|d|/max|ref| <= 1e-4.
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4


def x31_model():
    """VQ3R, hidden 512, inter 256, 16 experts, top-4, with exponent-31
    values in every kind's first stage (entries that codes select)."""
    model = ct.build(ct.Spec(hidden=512, inter=256, experts=16, top_k=4, layers=1, fmt="VQ3R", seed=77,
                             subnormals=False, keep_codes=False, **BALANCED))
    raw = model.books_raw.copy()
    S = ct.FMT_STAGES["VQ3R"]
    for kind in range(3):
        for e, d in ((3, 1), (40, 6), (200, 3)):
            # exponent 31, mantissa 0x11: +-2^16 * (1 + 17/1024) in the reference
            raw[kind * S, e, d] = np.uint16(0x7C00 | (0x8000 if e % 2 else 0) | 0x11)
    model.books_raw = raw
    return model


def test_x31_values_are_used():
    """The oracle's layer output moves when the exponent-31 entries are
    zeroed: the selected experts' rows do read them."""
    model = x31_model()
    x = np.random.default_rng(1).normal(size=512).astype(np.float32)
    y1 = po.LayerView(model, 0).moe_layer(x)[0]
    import copy
    m2 = copy.copy(model)
    raw = model.books_raw.copy()
    raw[((raw >> 10) & 0x1F) == 0x1F] = 0
    m2.books_raw = raw
    y2 = po.LayerView(m2, 0).moe_layer(x)[0]
    assert rel_err(y2, y1) > 1e-2


@pytest.mark.parametrize("path", ["auto", "mfma"])
def test_x31_decode(path):
    import warp_amd
    model = x31_model()
    ctx = open_ctx(model)
    ref = po.LayerView(model, 0)
    try:
        warp_amd.load_container_model(ctx, model)
        ctx.set_matvec_path(path)
        rng = np.random.default_rng(2)
        worst = 0.0
        for t in range(4):
            x = rng.normal(size=512).astype(np.float32)
            yr, ir, _, _ = ref.moe_layer(x)
            out = empty(512)
            idx, _ = ctx.moe_decode(0, dev(x), out, want_route=True)
            assert np.array_equal(idx, ir)
            e = rel_err(host(out), yr)
            worst = max(worst, e)
            assert np.all(np.isfinite(host(out))) and e <= TOL, (path, t, e)
        ctx.set_matvec_path("auto")
        log(f"exponent-31 codebooks, decode ({path} requested): worst rel err {worst:.2e}")
    finally:
        ctx.close()


@pytest.mark.parametrize("fp16", [False, True])
def test_x31_chunk(fp16):
    import warp_amd
    model = x31_model()
    ctx = open_ctx(model, max_tokens=12, prefill_fp16=fp16)
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(3).normal(size=(12, 512)).astype(np.float32)
        out, route, rw = ctx.moe_chunk_host(0, X)
        yr, rr, wr = po.LayerView(model, 0).moe_chunk(X)
        assert np.array_equal(route, rr)
        assert np.allclose(rw, wr, rtol=1e-6, atol=0)
        e = rel_err(out, yr)
        assert np.all(np.isfinite(out)) and e <= TOL, e
        log(f"exponent-31 codebooks, chunk of 12 (prefill_fp16={fp16}): routes bit-exact, rel err {e:.2e}")
    finally:
        ctx.close()


def test_x31_expert_ffn_and_matvec_on_mfma_path():
    import warp_amd
    model = x31_model()
    ctx = open_ctx(model)
    try:
        warp_amd.load_container_model(ctx, model)
        ctx.set_matvec_path("mfma")
        bT = po.books_T(model.books_raw)
        rec = np.frombuffer(model.layers[0].records[5], np.uint8)
        hdr = np.frombuffer(model.layers[0].records[5][:48], np.uint32)
        S, I, H = ct.FMT_STAGES["VQ3R"], 256, 512
        corr = int(hdr[8])

        def mat(kind):
            M = I if kind < 2 else H
            soff = [0, I, 2 * I][kind]
            return rec[int(hdr[5 + kind]):].copy(), rec[corr + 2 * soff: corr + 2 * (soff + M)].view(np.uint16).copy()

        x = np.random.default_rng(4).normal(size=H).astype(np.float32)
        g = po.vq_matvec("VQ3R", *mat(0), x, bT, 0, I, H)
        u = po.vq_matvec("VQ3R", *mat(1), x, bT, S, I, H)
        h = (np.array([po.lib().or_silu(float(v)) for v in g], np.float32) * u).astype(np.float32)
        yr = po.vq_matvec("VQ3R", *mat(2), h, bT, 2 * S, H, I)
        y = empty(H)
        ctx.expert_ffn(0, 5, dev(x), y)
        ctx.sync()
        assert rel_err(host(y), yr) <= TOL
        rec_dev = ctx.resident(0, 5)
        assert rec_dev
        yg = empty(I)
        ctx.vq_matvec(0, 0, rec_dev, dev(x), yg)
        assert rel_err(host(yg), g) <= TOL
        ctx.set_matvec_path("auto")
        log("exponent-31 codebooks: expert FFN and vq_matvec on the table kernel with mfma requested")
    finally:
        ctx.close()
