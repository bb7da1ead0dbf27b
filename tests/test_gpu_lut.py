"""The LUT expert matvec at shapes that exercise its work split: row groups
that span jobs (gate/up share one input), per-job groups (down), odd and
partial 64-row blocks, splits of a single 2-position chunk, and the
decode-then-dot path on the same inputs for comparison.

Bar: selection bit-exact, outputs max|d|/max|ref| <= 1e-4 against the oracle.
The tables are built on the matrix cores from x split into fp16 halves
(exact products, ~22 bits of x) and the rows are summed in a different order
from the oracle's (splits, then position parity); the logged errors are
~1e-7. The synthetic magnitudes keep the routed experts visible next to the
shared expert (checked on the oracle).
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err, routed_share
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4

SHAPES = [
    # partial last row block (96 = 64 + 32) and odd row-block counts; no shared expert
    dict(hidden=160, inter=96, experts=8, top_k=3, shared_bits=0),
    # gate/up: 8 jobs x 32 row blocks = 2 row groups spanning jobs; 1 chunk per split
    dict(hidden=1024, inter=2048, experts=12, top_k=8),
    # tiny: 8 row quads of gate/up (the row kernel's one-quad-per-XCD split) and 16 of down
    dict(hidden=64, inter=32, experts=4, top_k=2, shared_bits=0),
]


@pytest.mark.parametrize("fmt", ["VQ12", "VQ3R", "VQ2R"])
@pytest.mark.parametrize("shape", range(len(SHAPES)))
def test_lut_decode_and_matvec(fmt, shape):
    import warp_amd
    spec = ct.Spec(layers=1, fmt=fmt, seed=100 + shape, **SHAPES[shape], **BALANCED)
    model = ct.build(spec)
    ctx = open_ctx(model)
    try:
        warp_amd.load_container_model(ctx, model)
        log(f"[{fmt} {SHAPES[shape]}] loaded")
        lv = po.LayerView(model, 0)
        rng = np.random.default_rng(17)
        worst = {"auto": 0.0, "mfma": 0.0, "gather": 0.0}
        for t in range(3):
            x = rng.normal(size=spec.hidden).astype(np.float32)
            ro, ri, rw, _ = lv.moe_layer(x)
            if t == 0 and spec.shared_bits:
                assert routed_share(model, 0, x) > 0.05
            for path in ("auto", "mfma", "gather"):
                ctx.set_matvec_path(path)
                out = empty(spec.hidden)
                idx, w = ctx.moe_decode(0, dev(x), out, want_route=True)
                assert np.array_equal(idx, ri), (path, idx, ri)
                e = rel_err(host(out), ro)
                worst[path] = max(worst[path], e)
                assert e <= TOL, (path, t, e)
        log(f"[{fmt} {SHAPES[shape]}] moe_decode worst rel err lut {worst['auto']:.2e} "
            f"mfma {worst['mfma']:.2e} gather {worst['gather']:.2e}")

        S = ct.FMT_STAGES[fmt]
        bT = po.books_T(model.books_raw)
        for e in (0, spec.experts - 1):
            rec = ctx.resident(0, e)
            r = np.frombuffer(model.layers[0].records[e], np.uint8)
            hdr = np.frombuffer(model.layers[0].records[e][:48], np.uint32)
            for kind in range(3):
                M, N = (spec.inter, spec.hidden) if kind < 2 else (spec.hidden, spec.inter)
                x = rng.normal(size=N).astype(np.float32)
                off, corr = int(hdr[5 + kind]), int(hdr[8])
                soff = [0, spec.inter, 2 * spec.inter][kind]
                scale = r[corr + 2 * soff: corr + 2 * (soff + M)].view(np.uint16).copy()
                yr = po.vq_matvec(fmt, r[off:].copy(), scale, x, bT, kind * S, M, N)
                # auto: the gather kernel for one matrix; fused: the table kernel
                for path in ("auto", "fused"):
                    ctx.set_matvec_path(path)
                    y = empty(M)
                    ctx.vq_matvec(0, kind, rec, dev(x), y)
                    err = rel_err(host(y), yr)
                    assert err <= TOL, (e, kind, path, err)
        ctx.set_matvec_path("auto")
        log(f"[{fmt} {SHAPES[shape]}] vq_matvec (gather and table kernels) within bar")
    finally:
        ctx.close()
