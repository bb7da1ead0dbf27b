"""The MoE path behind the table: waste_register_hip_moe fills
waste_moe_kernels' moe_ffn_decode and moe_ffn_batch, and the engine calls
them with its own host tensors (warp_moe_args), as moe_layer and moe_chunk
would at their call sites (src/model.c:2713, 3512).

- Each golden spec (tests/golden/specs.py: VQ3R, VQ2R, VQ4P, SiTU, ties,
  latent; F32, Q8G and Q4G routers) goes through the registered slots with
  the model's f32 codebooks as the loader holds them, its trunk tensors and
  a fetch function standing in for bank_fetch; the outputs are compared
  with what the compiled reference's moe_layer and moe_chunk stored:
  selections and routes bit-exact, outputs within 1e-4 of max|ref|.
- A call the backend declines (a vector width it does not take) or fails
  (a selection whose records name different codebooks, E_BOOKS) goes to the
  slot's previous value with the same arguments; with the CPU default
  (NULL) the slot returns the negative code, and the engine's CPU path runs.
"""
import ctypes as C
import os
import struct

import numpy as np
import pytest

import container as ct
from gpu_util import log, rel_err
from oracle import pyoracle as po
from specs import SPECS

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4
INDEX_BITS = {"VQ3R": 8, "VQ2R": 8, "VQ4P": 6, "VQ12": 12}


class Engine:
    """The engine side of one model: its host tensors as waste_model holds
    them, and a fetch function over the container's records."""

    def __init__(self, model):
        from warp_amd import hip
        self.model = model
        self.spec = spec = model.spec
        self.books = po.books_flat(model.books_raw)         # f32, flushed as the loader flushes
        self.keep = []
        self.records = {(L, e): r for L in range(spec.layers) for e, r in enumerate(model.layers[L].records)}
        self.fetched = []

        def fetch(_user, layer, expert, dst):
            r = self.records.get((layer, expert))
            if r is None:
                return -1
            C.memmove(dst, r, len(r))
            self.fetched.append((layer, expert))
            return 0
        self.fetch = hip.FETCH_FN(fetch)
        self.identity = C.c_int(0)                           # the model's address stands for waste_model*

    def tensor(self, t, q=None):
        from warp_amd import hip
        tt = hip.TrunkTensor()
        if q is None:
            a = np.ascontiguousarray(t, np.float32)
            self.keep.append(a)
            tt.data = a.ctypes.data
        else:
            pl, sc, rb, bits, group = q
            pl, sc = np.ascontiguousarray(pl), np.ascontiguousarray(sc)
            self.keep += [pl, sc]
            tt.q, tt.qs, tt.rowbytes, tt.bits, tt.group = pl.ctypes.data, sc.ctypes.data, rb, bits, group
        return tt

    def args(self, L, x, out, route, rw):
        from warp_amd import hip
        spec, lay = self.spec, self.model.layers[L]
        S = ct.FMT_STAGES[spec.fmt]
        a = hip.MoeArgs()
        a.model = C.addressof(self.identity)
        a.layer, a.n_layers = L, spec.layers
        a.hidden, a.moe_inter, a.n_experts, a.top_k = spec.hidden, spec.inter, spec.experts, spec.top_k
        a.latent_dim, a.latent_norm, a.norm_eps = spec.latent, int(spec.latent_norm), 1e-5
        a.renorm, a.routed_scale = int(spec.renorm), spec.routed_scale
        a.act_situ, a.situ_beta, a.situ_linear_beta = int(spec.act == "situ"), spec.situ_beta, spec.situ_lbeta
        a.index_bits, a.stages, a.cb_entries, a.vec_dim = INDEX_BITS[spec.fmt], S, ct.FMT_ENTRIES[spec.fmt], 8
        a.codebooks, a.n_books, a.cb_base = self.books.ctypes.data, self.books.shape[0], L * 3 * S
        a.router = self.tensor(lay.router, lay.router_q)
        if lay.bias is not None:
            self.keep.append(lay.bias)
            a.bias = lay.bias.ctypes.data
        for k, (pl, sc, rb) in enumerate(lay.shared):
            a.shared[k] = self.tensor(None, (pl, sc, rb, spec.shared_bits, spec.shared_group))
        a.inter_shared = spec.inter * spec.n_shared
        if lay.latent is not None:
            dq, uq, nw = lay.latent
            a.latent[0], a.latent[1] = self.tensor(None, dq), self.tensor(None, uq)
            if nw is not None:
                self.keep.append(nw)
                a.latent_norm_w = nw.ctypes.data
        a.rec_bytes = self.model.rec_bytes
        a.cache_bytes = spec.layers * spec.experts * self.model.rec_bytes
        a.fetch, a.fetch_user = self.fetch, None
        a.n_tokens = x.shape[0] if x.ndim == 2 else 1
        for name, arr in (("x", x), ("out", out), ("route", route), ("rw", rw)):
            setattr(a, name, arr.ctypes.data if arr is not None else None)
        return a


def registered(prev_decode=None, prev_batch=None):
    import warp_amd
    from warp_amd import hip
    t = hip.MoeKernels()
    if prev_decode is not None:
        t.moe_ffn_decode = prev_decode
    if prev_batch is not None:
        t.moe_ffn_batch = prev_batch
    assert warp_amd.lib().waste_register_hip_moe(C.byref(t)) == b"HIP gfx950"
    assert t.on_device == 1
    return t


def stats():
    import warp_amd
    d, f = C.c_uint64(), C.c_uint64()
    warp_amd.lib().warp_hip_moe_table_stats(C.byref(d), C.byref(f))
    return d.value, f.value


@pytest.mark.parametrize("name", sorted(SPECS))
def test_slots_against_reference_outputs(name):
    import warp_amd
    spec = SPECS[name]
    model = ct.build(spec)
    g = dict(np.load(os.path.join(HERE, f"{name}.npz")))
    eng = Engine(model)
    t = registered()
    d0, f0 = stats()
    worst = 0.0
    try:
        for L in range(spec.layers):
            for i in range(g[f"L{L}_x"].shape[0]):
                x = np.ascontiguousarray(g[f"L{L}_x"][i])
                out = np.empty(spec.hidden, np.float32)
                route = np.empty(spec.top_k, np.int32)
                rw = np.empty(spec.top_k, np.float32)
                a = eng.args(L, x, out, route, rw)
                assert t.moe_ffn_decode(C.byref(a)) == 0
                assert np.array_equal(route, g[f"L{L}_idx"][i]), (name, L, i)
                e = rel_err(out, g[f"L{L}_out"][i])
                worst = max(worst, e)
                assert e <= TOL, (name, L, i, e)
            X = np.ascontiguousarray(g[f"L{L}_chunk_x"])
            out = np.empty_like(X)
            route = np.empty((X.shape[0], spec.top_k), np.int32)
            rw = np.empty((X.shape[0], spec.top_k), np.float32)
            a = eng.args(L, X, out, route, rw)
            assert t.moe_ffn_batch(C.byref(a)) == 0
            assert np.array_equal(route, g[f"L{L}_chunk_route"]), (name, L)
            assert np.allclose(rw, g[f"L{L}_chunk_w"], rtol=1e-5, atol=0)
            e = rel_err(out, g[f"L{L}_chunk_out"])
            worst = max(worst, e)
            assert e <= TOL, (name, L, e)
        d1, f1 = stats()
        assert f1 == f0 and d1 - d0 == spec.layers * (g["L0_x"].shape[0] + 1)
        # every record came through the engine's fetch function, each once
        assert len(eng.fetched) == len(set(eng.fetched)) > 0
    finally:
        warp_amd.lib().waste_hip_release_host_buffers()
    log(f"[{name}] moe_ffn_decode / moe_ffn_batch through the registered table: selections bit-exact, "
        f"worst rel err {worst:.2e} against the reference's stored outputs")


def test_declined_and_failed_calls_fall_back():
    import warp_amd
    from warp_amd import hip
    spec = SPECS["vq3r_f32"]
    model = ct.build(spec)
    g = dict(np.load(os.path.join(HERE, "vq3r_f32.npz")))
    eng = Engine(model)
    calls = []

    def cpu_decode(p):
        calls.append(("decode", C.addressof(p.contents)))
        return 0

    def cpu_batch(p):
        calls.append(("batch", C.addressof(p.contents)))
        return 0
    prev_d, prev_b = hip.MOE_SLOT(cpu_decode), hip.MOE_SLOT(cpu_batch)
    try:
        t = registered(prev_d, prev_b)
        x = np.ascontiguousarray(g["L0_x"][0])
        out = np.empty(spec.hidden, np.float32)
        route = np.empty(spec.top_k, np.int32)
        # declined: a vector width this backend does not take
        a = eng.args(0, x, out, route, None)
        a.vec_dim = 4
        assert t.moe_ffn_decode(C.byref(a)) == 0 and calls == [("decode", C.addressof(a))]
        X = np.ascontiguousarray(g["L0_chunk_x"])
        b = eng.args(0, X, np.empty_like(X), np.empty((X.shape[0], spec.top_k), np.int32), None)
        b.vec_dim = 4
        assert t.moe_ffn_batch(C.byref(b)) == 0 and calls[-1] == ("batch", C.addressof(b))
        # failed: the selection's records name different codebooks
        picked = [int(e) for e in g["L0_idx"][0]]
        S = ct.FMT_STAGES[spec.fmt]
        rec = bytearray(eng.records[(0, picked[1])])
        struct.pack_into("<H", rec, 10, 3 * S)               # layer 1's codebook base
        eng.records[(0, picked[1])] = bytes(rec)
        a = eng.args(0, x, out, route, None)
        assert t.moe_ffn_decode(C.byref(a)) == 0 and calls[-1] == ("decode", C.addressof(a))
        # with the CPU default the slot returns the code; the engine runs its CPU path
        warp_amd.lib().waste_hip_release_host_buffers()
        t2 = registered()
        a = eng.args(0, x, out, route, None)
        assert t2.moe_ffn_decode(C.byref(a)) == warp_amd.E_BOOKS
        a.vec_dim = 4
        assert t2.moe_ffn_decode(C.byref(a)) == warp_amd.E_ARG
    finally:
        warp_amd.lib().waste_hip_release_host_buffers()
        registered()                                          # no Python callback left as a previous slot
    log("declined (vector width) and failed (E_BOOKS) slot calls reach the previous slot / return the code")
