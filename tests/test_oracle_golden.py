"""The oracle against golden vectors written by the compiled reference
(tests/golden/make_golden.py) on the synthetic containers of specs.py.
Every comparison is bit for bit."""
import os

import numpy as np
import pytest

import container as ct
from oracle import pyoracle as po
from specs import SPECS

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(HERE, f"{name}.npz")))


@pytest.fixture(scope="module", params=sorted(SPECS))
def case(request):
    name = request.param
    spec = SPECS[name]
    model = ct.build(spec)
    return name, spec, model, load(name)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_generator_reproduces_fixture_bytes(case):
    name, spec, model, g = case
    assert ct.digest(model) == g["digest"].tobytes().decode(), f"{name}: container generator drifted"


def test_moe_layer_bitexact(case):
    name, spec, model, g = case
    for L in range(spec.layers):
        lv = po.LayerView(model, L)
        for t in range(g[f"L{L}_x"].shape[0]):
            out, idx, w, logits = lv.moe_layer(g[f"L{L}_x"][t])
            assert np.array_equal(bits(logits), bits(g[f"L{L}_logits"][t])), (name, L, t)
            assert np.array_equal(idx, g[f"L{L}_idx"][t]), (name, L, t)
            assert np.array_equal(bits(out), bits(g[f"L{L}_out"][t])), (name, L, t)


def test_weights_follow_unbiased_scores(case):
    """w = renorm(score[idx]) * scale, scores being the reference's sigmoids."""
    name, spec, model, g = case
    for L in range(spec.layers):
        for t in range(g[f"L{L}_x"].shape[0]):
            idx, w, sc = po.route(g[f"L{L}_logits"][t], model.layers[L].bias, spec.top_k, 0,
                                  int(spec.renorm), spec.routed_scale)
            assert np.array_equal(bits(sc), bits(g[f"L{L}_scores"][t]))
            assert np.array_equal(idx, g[f"L{L}_idx"][t])


def test_moe_chunk_bitexact(case):
    name, spec, model, g = case
    for L in range(spec.layers):
        out, route, rw = po.LayerView(model, L).moe_chunk(g[f"L{L}_chunk_x"])
        assert np.array_equal(route, g[f"L{L}_chunk_route"])
        assert np.array_equal(bits(rw), bits(g[f"L{L}_chunk_w"]))
        assert np.array_equal(bits(out), bits(g[f"L{L}_chunk_out"]))


def test_vq_matvec_and_lut_bitexact(case):
    name, spec, model, g = case
    S, EN = ct.FMT_STAGES[spec.fmt], ct.FMT_ENTRIES[spec.fmt]
    bT = po.books_T(model.books_raw)
    Hx = spec.latent or spec.hidden                  # the experts' width
    for L in range(spec.layers):
        rec = np.frombuffer(model.layers[L].records[1], np.uint8)
        hdr = np.frombuffer(model.layers[L].records[1][:48], np.uint32)
        for kind in range(3):
            M, N = (spec.inter, Hx) if kind < 2 else (Hx, spec.inter)
            soff = [0, spec.inter, 2 * spec.inter][kind]
            corr = int(hdr[8])
            scale = rec[corr + 2 * soff: corr + 2 * (soff + M)].view(np.uint16).copy()
            y = po.vq_matvec(spec.fmt, rec[int(hdr[5 + kind]):].copy(), scale, g[f"L{L}_mv{kind}_x"], bT,
                             L * 3 * S + kind * S, M, N, fused=1)
            assert np.array_equal(bits(y), bits(g[f"L{L}_mv{kind}_y"])), (name, L, kind)
        x = g[f"L{L}_lut_x"]
        lut = np.empty((Hx // 8) * S * EN, np.float32)
        po.lib().or_lutb_range(0, Hx // 8, lut.ctypes.data, bT.ctypes.data, x.ctypes.data,
                               L * 3 * S, S, EN, 8, 1)
        assert np.array_equal(bits(lut), bits(g[f"L{L}_lut"]))


def test_ties_go_to_the_lowest_id():
    g = load("vq3r_ties")
    a, b = SPECS["vq3r_ties"].dup_rows
    seen = 0
    for L in range(SPECS["vq3r_ties"].layers):
        for t in range(g[f"L{L}_x"].shape[0]):
            lg, idx = g[f"L{L}_logits"][t], list(g[f"L{L}_idx"][t])
            assert lg[a] == lg[b]
            if b in idx:
                assert a in idx and idx.index(a) < idx.index(b)
                seen += 1
            if a in idx:
                seen += 1
    assert seen, "the tie case never reached the selection"


def test_kda_step_bitexact_against_the_reference():
    """The oracle's KDA step (or_kda_step) against the compiled reference's
    waste_kda_step outputs in tests/golden/kda.npz (make_kda.py), over
    several steps and shapes: state and outputs bit for bit."""
    g = load("kda")
    n = 0
    while f"c{n}_q" in g:
        S, o = po.kda_forward(g[f"c{n}_q"], g[f"c{n}_k"], g[f"c{n}_v"], g[f"c{n}_g"], g[f"c{n}_beta"], g[f"c{n}_S0"])
        assert np.array_equal(bits(S), bits(g[f"c{n}_S"])), n
        assert np.array_equal(bits(o), bits(g[f"c{n}_o"])), n
        n += 1
    assert n == 3
