"""The benchmark configurations as parity cases, at their real shapes, through
the C ABI against the oracle (synthetic data per the configurations' rules:
N(0,1) activations, N(0, 0.02) fp16 codebooks and fp32 routers, uniform
codes, U(0.01, 0.05) row scales).

- single expert, decode: H 2304, I 1024, every matrix on both matvec kernels;
- Kimi-Linear layer, decode: E 256, top-8, Q8G g32 shared expert;
- Kimi-Linear prefill: 64 tokens against the oracle's moe_chunk, and 512
  tokens with a Zipf-like skew through properties that hold at any size
  (token order does not change any token's result, bit for bit; each token
  equals its own single-token decode within the bar).

The Kimi-Linear cases run with both routings: the reference's sigmoid and
the softmax the configurations name (an extension the reference does not
have; the oracle's softmax is pinned against float64 in
test_oracle_math.py). Decode covers the table kernel, whose gate/up launch
routes the token itself, and the decode-then-dot kernel after the routing
launch; prefill routes each token in its own block.

Only the experts routing can select get records (the rest are never read);
their bias is lifted so that selection stays among them, as in the
benchmark. The K3-scale miss path is covered at reduced size by
test_gpu_cache.py (its invariants do not depend on the shape).
"""
import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err, routed_share
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-4
KIMI = dict(hidden=2304, inter=1024, experts=256, top_k=8, layers=1, shared_bits=8, shared_group=32,
            subnormals=False, keep_codes=False, **BALANCED)


def lifted(spec_kw, ids, lift):
    """A model whose experts `ids` alone have records, their bias raised by lift[i]."""
    model = ct.build(ct.Spec(materialize=tuple(int(i) for i in ids), **spec_kw))
    lay = model.layers[0]
    b = np.zeros(spec_kw["experts"], np.float32) if lay.bias is None else lay.bias.copy()
    b[np.asarray(ids)] += np.asarray(lift, np.float32)
    lay.bias = b
    return model


@pytest.mark.parametrize("fmt", ["VQ12", "VQ3R"])
def test_config1_single_expert(fmt):
    import warp_amd
    spec = ct.Spec(hidden=2304, inter=1024, experts=2, top_k=1, layers=1, fmt=fmt, seed=1, subnormals=False,
                   keep_codes=False, **BALANCED)
    model = ct.build(spec)
    ctx = open_ctx(model)
    try:
        warp_amd.load_container_model(ctx, model)
        S = ct.FMT_STAGES[fmt]
        bT = po.books_T(model.books_raw)
        rng = np.random.default_rng(0)
        r = np.frombuffer(model.layers[0].records[1], np.uint8)
        hdr = np.frombuffer(model.layers[0].records[1][:48], np.uint32)
        rec = ctx.resident(0, 1)
        for kind in range(3):
            M, N = (spec.inter, spec.hidden) if kind < 2 else (spec.hidden, spec.inter)
            x = rng.normal(size=N).astype(np.float32)
            off, corr = int(hdr[5 + kind]), int(hdr[8])
            soff = [0, spec.inter, 2 * spec.inter][kind]
            scale = r[corr + 2 * soff: corr + 2 * (soff + M)].view(np.uint16).copy()
            yr = po.vq_matvec(fmt, r[off:].copy(), scale, x, bT, kind * S, M, N)
            for path in ("auto", "mfma", "fused"):
                ctx.set_matvec_path(path)
                y = empty(M)
                ctx.vq_matvec(0, kind, rec, dev(x), y)
                e = rel_err(host(y), yr)
                assert e <= TOL, (kind, path, e)
        # the whole expert FFN (warp_hip_expert_ffn): the oracle's gate and up
        # matvecs, SiLU(gate) * up, the down matvec
        S0 = [0, S, 2 * S]
        mats = []
        for kind in range(3):
            M, N = (spec.inter, spec.hidden) if kind < 2 else (spec.hidden, spec.inter)
            soff = [0, spec.inter, 2 * spec.inter][kind]
            corr = int(hdr[8])
            mats.append((r[int(hdr[5 + kind]):].copy(), r[corr + 2 * soff: corr + 2 * (soff + M)].view(np.uint16).copy(),
                         M, N))
        for t in range(3):
            x = rng.normal(size=spec.hidden).astype(np.float32)
            g = po.vq_matvec(fmt, mats[0][0], mats[0][1], x, bT, S0[0], spec.inter, spec.hidden)
            u = po.vq_matvec(fmt, mats[1][0], mats[1][1], x, bT, S0[1], spec.inter, spec.hidden)
            h = np.array([po.lib().or_silu(float(v)) for v in g], np.float32) * u
            yr = po.vq_matvec(fmt, mats[2][0], mats[2][1], h.astype(np.float32), bT, S0[2], spec.hidden, spec.inter)
            for path in ("auto", "mfma", "fused"):
                ctx.set_matvec_path(path)
                y = empty(spec.hidden)
                ctx.expert_ffn(0, 1, dev(x), y)
                ctx.sync()
                e = rel_err(host(y), yr)
                assert e <= TOL, (t, path, e)
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.expert_ffn(0, 2, dev(x), empty(spec.hidden))      # expert 2 of 2 does not exist
        assert ei.value.code == warp_amd.E_ARG
        ctx.set_matvec_path("auto")
        log(f"config 1 ({fmt}): gate, up, down and the whole expert FFN within the bar on the gather (auto), "
            f"matrix-core and table (fused) kernels")
    finally:
        ctx.close()


ACTS = {"sigmoid": 0, "softmax": 1}


@pytest.mark.parametrize("act", sorted(ACTS))
def test_config2_kimi_layer(act):
    import warp_amd
    ids = np.arange(3, 256, 8)[:24]                 # 24 experts spread over the id range
    model = lifted(dict(KIMI, fmt="VQ12", seed=2), ids, np.full(len(ids), 1.0))
    ctx = open_ctx(model, cache_slots=len(ids), router_act=ACTS[act])
    try:
        warp_amd.load_container_model(ctx, model)
        lv = po.LayerView(model, 0, router_act=ACTS[act])
        rng = np.random.default_rng(3)
        worst = 0.0
        for t in range(4):
            x = rng.normal(size=KIMI["hidden"]).astype(np.float32)
            ro, ri, rw, _ = lv.moe_layer(x)
            if t == 0:
                share = routed_share(model, 0, x)
                assert share > 0.05, share
            outs = {}
            for path in ("auto", "mfma", "gather"):
                ctx.set_matvec_path(path)
                out = empty(KIMI["hidden"])
                idx, w = ctx.moe_decode(0, dev(x), out, want_route=True)
                assert np.array_equal(idx, ri), (path, idx, ri)
                outs[path] = host(out)
                e = rel_err(outs[path], ro)
                worst = max(worst, e)
                assert e <= TOL, (t, path, e)
        ctx.set_matvec_path("auto")
        log(f"config 2 ({act}): Kimi-Linear layer (E 256, top-8, Q8G g32 shared) worst rel err {worst:.2e}; routed "
            f"share of the output {share:.2f}; LUT vs MFMA decode max|d| {np.abs(outs['auto'] - outs['mfma']).max():.2e}")
    finally:
        ctx.close()


def zipf_model(fmt, seed, n=48, s=1.1, act="sigmoid"):
    """n experts with records, biases falling with rank so that token counts
    per expert follow a Zipf-like skew under the reference's own selection
    rule (softmax scores spread about 20x less than sigmoid ones at these
    logits, so their bias steps are smaller by as much)."""
    ids = np.random.default_rng(seed).permutation(256)[:n]
    step = 0.06 if act == "sigmoid" else 0.003
    lift = 1.0 + step * (np.arange(n, dtype=np.float64) + 1.0) ** -s
    return lifted(dict(KIMI, fmt=fmt, seed=seed), ids, lift), ids


@pytest.mark.parametrize("act", sorted(ACTS))
def test_config3_prefill_64_against_oracle(act):
    import warp_amd
    model, _ = zipf_model("VQ12", 4, act=act)
    ctx = open_ctx(model, max_tokens=64, cache_slots=48, router_act=ACTS[act])
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(5).normal(size=(64, KIMI["hidden"])).astype(np.float32)
        assert routed_share(model, 0, X[0]) > 0.05
        out, route, rw = ctx.moe_chunk_host(0, X)
        ro, rr, rrw = po.LayerView(model, 0, router_act=ACTS[act]).moe_chunk(X)
        assert np.array_equal(route, rr)
        assert np.allclose(rw, rrw, rtol=1e-5, atol=0), float(np.max(np.abs(rw - rrw) / np.abs(rrw)))
        e = rel_err(out, ro)
        assert e <= TOL, e
        counts = np.bincount(route.ravel(), minlength=256)
        assert len(np.unique(route)) > 8, "selection did not spread over the lifted experts"
        log(f"config 3 ({act}), 64 tokens: rel err {e:.2e}; tokens on the 5 busiest experts {sorted(counts)[-5:]}; "
            f"{len(np.unique(route))} distinct experts")
    finally:
        ctx.close()


@pytest.mark.parametrize("act", sorted(ACTS))
def test_config3_prefill_512_properties(act):
    import warp_amd
    model, _ = zipf_model("VQ12", 6, act=act)
    T = 512
    ctx = open_ctx(model, max_tokens=T, cache_slots=48, router_act=ACTS[act])
    try:
        warp_amd.load_container_model(ctx, model)
        X = np.random.default_rng(7).normal(size=(T, KIMI["hidden"])).astype(np.float32)
        out, route, _ = ctx.moe_chunk_host(0, X)
        perm = np.random.default_rng(8).permutation(T)
        out_p, route_p, _ = ctx.moe_chunk_host(0, X[perm])
        assert np.array_equal(route_p, route[perm])
        assert np.array_equal(out_p.view(np.uint32), out[perm].view(np.uint32)), "token order changed a result"
        worst = 0.0
        for t in range(0, T, 37):
            o = empty(KIMI["hidden"])
            idx, _ = ctx.moe_decode(0, dev(X[t]), o, want_route=True)
            assert np.array_equal(idx, route[t]), t
            e = rel_err(host(o), out[t])
            worst = max(worst, e)
            assert e <= TOL, (t, e)
        counts = np.bincount(route.ravel(), minlength=256)
        log(f"config 3 ({act}), 512 tokens: order-invariant bit for bit; decode vs chunk worst {worst:.2e}; "
            f"pairs on the 5 busiest experts {sorted(counts)[-5:]} of {T * 8}")
    finally:
        ctx.close()
