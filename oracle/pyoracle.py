"""ctypes bindings for liboracle.so (the CPU restatement in oracle.c).

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker, never by the shipped package.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libwaste_ref.so")

FMT = {"VQ3R": 4, "VQ2R": 5, "VQ4P": 8, "VQ12": 9}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built (make -C oracle)")
        _lib = C.CDLL(LIB)
        _declare(_lib)
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def _declare(L):
    vp, i, f, sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
    sig = {
        "or_f16_keep": (f, [C.c_uint16]), "or_f16_flush": (f, [C.c_uint16]),
        "or_silu": (f, [f]), "or_situ_pair": (f, [f, f, f, f]),
        "or_index_bytes": (sz, [i, i, i]),
        "or_pack_indices": (None, [i, vp, i, i, vp]),
        "or_code_at": (C.c_uint, [i, vp, i, i, i, i]),
        "or_books_decode": (None, [vp, i, i, i, vp, vp]),
        "or_decode_weights": (None, [i, vp, vp, vp, i, i, i, vp]),
        "or_lutb_range": (None, [i, i, vp, vp, vp, i, i, i, i, i]),
        "or_vq_apply": (None, [i, vp, vp, vp, vp, i, i]),
        "or_vq_quant_lut": (None, [vp, i, i, i, vp, vp]),
        "or_vq_apply_p6": (None, [vp, vp, vp, vp, vp, i, i]),
        "or_vq_matvec": (None, [i, vp, vp, vp, vp, vp, i, i, i, i, vp, vp, vp]),
        "or_dotf": (f, [vp, vp, i]),
        "or_mvq_rows_f32": (None, [i, i, vp, vp, vp, vp, i, i, i, i, sz, i]),
        "or_mmq_rows": (None, [i, i, vp, vp, vp, vp, i, i, i, i, sz]),
        "or_route": (None, [vp, vp, i, i, i, i, f, vp, vp, vp]),
        "or_moe_layer": (i, [vp, vp, vp, vp, vp, vp]),
        "or_moe_chunk": (i, [vp, vp, vp, i, vp, vp]),
        "or_expert_ffn": (None, [vp, vp, vp, vp, vp, vp, vp, vp, vp]),
        "or_vq_encode": (None, [vp, i, vp, i, i, i, vp]),
        "or_crc32": (C.c_uint32, [vp, sz]),
        "or_expf_mismatches": (C.c_uint64, [C.c_uint32, C.c_uint64, i, vp]),
        "or_expf_decreases": (C.c_uint64, [i]),
        "or_kda_step": (None, [i, i, i, vp, vp, vp, vp, vp, vp, vp]),
        "or_rmsnorm": (None, [vp, vp, vp, i, f]),
        "or_expf_array": (None, [vp, vp, C.c_long]),
        "or_sigmoid_array": (None, [vp, vp, C.c_long]),
        "or_record_check": (i, [vp, sz, i, i, i, i, i, vp, i]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


class OrLayer(C.Structure):
    _fields_ = [
        ("fmt", C.c_int), ("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int),
        ("top_k", C.c_int), ("renorm", C.c_int), ("routed_scale", C.c_float),
        ("router_act", C.c_int), ("act_situ", C.c_int), ("situ_beta", C.c_float),
        ("situ_lbeta", C.c_float), ("booksT", C.c_void_p), ("router", C.c_void_p),
        ("router_q", C.c_void_p), ("router_s", C.c_void_p), ("router_rowbytes", C.c_size_t),
        ("router_bits", C.c_int), ("router_group", C.c_int),
        ("bias", C.c_void_p), ("recs", C.c_void_p),
        ("sh_q", C.c_void_p * 3), ("sh_s", C.c_void_p * 3), ("sh_rowbytes", C.c_size_t * 3),
        ("sh_group", C.c_int), ("sh_bits", C.c_int), ("sh_inter", C.c_int),
        ("fused_lutb", C.c_int), ("mvq_isa", C.c_int),
        ("latent", C.c_int), ("lat_q", C.c_void_p * 2), ("lat_s", C.c_void_p * 2), ("lat_rowbytes", C.c_size_t * 2),
        ("lat_bits", C.c_int), ("lat_group", C.c_int), ("lat_norm", C.c_void_p), ("eps", C.c_float),
    ]


def books_T(books_raw: np.ndarray) -> np.ndarray:
    nb, E, vd = books_raw.shape
    out = np.empty((nb, vd, E), np.float32)
    lib().or_books_decode(_p(np.ascontiguousarray(books_raw)), nb, E, vd, None, _p(out))
    return out


def books_flat(books_raw: np.ndarray) -> np.ndarray:
    nb, E, vd = books_raw.shape
    out = np.empty((nb, E, vd), np.float32)
    lib().or_books_decode(_p(np.ascontiguousarray(books_raw)), nb, E, vd, _p(out), None)
    return out


class LayerView:
    """An or_layer over one layer of a tests/golden/container.Model. Keeps
    every array it points at alive."""

    def __init__(self, model, L: int, router_act: int = 0, fused_lutb: int = 1, mvq_isa: int = 2):
        spec = model.spec
        lay = model.layers[L]
        self.keep = []
        self.booksT = books_T(model.books_raw)
        # experts without a record (not materialised) are NULL: the oracle reads
        # only the records of the experts a token selects
        self.recs = [None if r is None else np.frombuffer(r, dtype=np.uint8) for r in lay.records]
        self.rec_ptrs = (C.c_void_p * len(self.recs))(*[None if r is None else r.ctypes.data for r in self.recs])
        st = OrLayer()
        st.fmt = FMT[spec.fmt]
        st.hidden, st.inter, st.n_experts, st.top_k = spec.hidden, spec.inter, spec.experts, spec.top_k
        st.renorm = int(spec.renorm)
        st.routed_scale = spec.routed_scale
        st.router_act = router_act
        st.act_situ = int(spec.act == "situ")
        st.situ_beta, st.situ_lbeta = spec.situ_beta, spec.situ_lbeta
        st.booksT = self.booksT.ctypes.data
        if lay.router_q is None:
            self.router = np.ascontiguousarray(lay.router, dtype=np.float32)
            st.router = self.router.ctypes.data
        else:
            pl, sc, rb, bits, group = lay.router_q
            self.keep += [pl, sc]
            st.router = None
            st.router_q, st.router_s = pl.ctypes.data, sc.ctypes.data
            st.router_rowbytes, st.router_bits, st.router_group = rb, bits, group
        self.bias = lay.bias
        st.bias = lay.bias.ctypes.data if lay.bias is not None else None
        st.recs = C.cast(self.rec_ptrs, C.c_void_p)
        if lay.shared:
            for k, (pl, sc, rb) in enumerate(lay.shared):
                self.keep += [pl, sc]
                st.sh_q[k] = pl.ctypes.data
                st.sh_s[k] = sc.ctypes.data
                st.sh_rowbytes[k] = rb
            st.sh_group, st.sh_bits = spec.shared_group, spec.shared_bits
            st.sh_inter = spec.inter * spec.n_shared
        st.fused_lutb, st.mvq_isa = fused_lutb, mvq_isa
        st.eps = 1e-5                           # the containers' rms_norm_eps
        if getattr(lay, "latent", None) is not None:
            dq, uq, nw = lay.latent
            st.latent = spec.latent
            for k, q in enumerate((dq, uq)):
                self.keep += [q[0], q[1]]
                st.lat_q[k], st.lat_s[k], st.lat_rowbytes[k] = q[0].ctypes.data, q[1].ctypes.data, q[2]
            st.lat_bits, st.lat_group = dq[3], dq[4]
            if nw is not None:
                self.keep.append(nw)
                st.lat_norm = nw.ctypes.data
        self.st = st

    def moe_layer(self, x: np.ndarray):
        st = self.st
        out = np.empty(st.hidden, np.float32)
        idx = np.empty(st.top_k, np.int32)
        w = np.empty(st.top_k, np.float32)
        logits = np.empty(st.n_experts, np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        rc = lib().or_moe_layer(C.byref(st), _p(x), _p(out), _p(idx), _p(w), _p(logits))
        assert rc == 0
        return out, idx, w, logits

    def moe_chunk(self, X: np.ndarray):
        st = self.st
        X = np.ascontiguousarray(X, dtype=np.float32)
        nT = X.shape[0]
        out = np.empty((nT, st.hidden), np.float32)
        route = np.empty((nT, st.top_k), np.int32)
        rw = np.empty((nT, st.top_k), np.float32)
        rc = lib().or_moe_chunk(C.byref(st), _p(X), _p(out), nT, _p(route), _p(rw))
        assert rc == 0
        return out, route, rw


def vq_matvec(fmt: str, idx: np.ndarray, scale: np.ndarray, x: np.ndarray, booksT: np.ndarray,
              cb_base: int, M: int, N: int, fused: int = 1) -> np.ndarray:
    S = {"VQ3R": 3, "VQ2R": 2, "VQ4P": 4, "VQ12": 2}[fmt]
    E = {"VQ3R": 256, "VQ2R": 256, "VQ4P": 64, "VQ12": 4096}[fmt]
    nv = N // 8
    y = np.empty(M, np.float32)
    lut = np.empty(nv * S * E, np.float32)
    q8 = np.empty(nv * S * E, np.int8)
    qs = np.empty(nv // 32 + 2, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lib().or_vq_matvec(FMT[fmt], _p(y), _p(idx), _p(scale), _p(x), _p(booksT), cb_base, M, N,
                       fused, _p(lut), _p(q8), _p(qs))
    return y


def decode_weights(fmt: str, idx: np.ndarray, scale: np.ndarray, books: np.ndarray, cb_base: int,
                   M: int, N: int) -> np.ndarray:
    W = np.empty((M, N), np.float32)
    lib().or_decode_weights(FMT[fmt], _p(idx), _p(scale), _p(books), cb_base, M, N, _p(W))
    return W


def route(logits, bias, K, act=0, renorm=1, routed_scale=1.0):
    logits = np.ascontiguousarray(logits, np.float32)
    E = logits.shape[0]
    idx = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    sc = np.empty(E, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().or_route(_p(logits), _p(b), E, K, act, renorm, routed_scale, _p(idx), _p(w), _p(sc))
    return idx, w, sc


# ---- the compiled reference (present only where /root/reference is) -------------

class Ref:
    """oracle/_ref/libwaste_ref.so over one container directory."""

    def __init__(self, container_dir: str, cache_bytes: int = 0, n_threads: int = 1):
        if not os.path.exists(REF_LIB):
            raise RuntimeError(f"{REF_LIB} is not built")
        self.L = C.CDLL(REF_LIB)
        L = self.L
        vp, i = C.c_void_p, C.c_int
        L.ref_open.restype = vp
        L.ref_open.argtypes = [C.c_char_p, C.c_size_t, C.c_int]
        L.ref_threads.restype = C.c_int
        L.ref_close.argtypes = [vp]
        L.ref_backend.restype = C.c_char_p
        L.ref_moe_layer.restype = i
        L.ref_moe_layer.argtypes = [vp, i, vp, vp, vp, vp, vp]
        L.ref_moe_chunk.restype = i
        L.ref_moe_chunk.argtypes = [vp, i, vp, vp, i, vp, vp]
        L.ref_build_lut.argtypes = [vp, i, i, vp, i, vp]
        L.ref_vq_matvec.restype = i
        L.ref_vq_matvec.argtypes = [vp, i, i, i, vp, vp]
        L.ref_pool_reset.restype = None
        L.ref_save_usage.restype = i
        L.ref_save_usage.argtypes = [vp, C.c_char_p]
        L.ref_expert_ffn.restype = i
        L.ref_expert_ffn.argtypes = [vp, i, i, vp, vp]
        L.ref_trunk_matvec.restype = i
        L.ref_trunk_matvec.argtypes = [vp, C.c_char_p, vp, vp, i, i]
        L.ref_record_check.restype = i
        L.ref_record_check.argtypes = [vp, i, i, vp, i]
        L.ref_n_books.restype = i
        L.ref_n_books.argtypes = [vp]
        self.m = L.ref_open(container_dir.encode(), cache_bytes, n_threads)
        if not self.m:
            raise RuntimeError(f"reference refused {container_dir}")

    def close(self, reset_pool=False):
        """reset_pool: also end the reference's process-wide thread pool, so a
        model opened next gets a pool of its own n_threads."""
        if self.m:
            self.L.ref_close(self.m)
            self.m = None
        if reset_pool:
            self.L.ref_pool_reset()

    def backend(self) -> str:
        return self.L.ref_backend().decode()

    def threads(self) -> int:
        return self.L.ref_threads()

    def moe_layer(self, L, x, E, K, H):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(H, np.float32)
        idx = np.empty(K, np.int32)
        logits = np.empty(E, np.float32)
        scores = np.empty(E, np.float32)
        rc = self.L.ref_moe_layer(self.m, L, _p(x), _p(out), _p(idx), _p(logits), _p(scores))
        assert rc == 0, rc
        return out, idx, logits, scores

    def moe_chunk(self, L, X, K, H):
        X = np.ascontiguousarray(X, np.float32)
        nT = X.shape[0]
        out = np.empty((nT, H), np.float32)
        route = np.empty((nT, K), np.int32)
        rw = np.empty((nT, K), np.float32)
        rc = self.L.ref_moe_chunk(self.m, L, _p(X), _p(out), nT, _p(route), _p(rw))
        assert rc == 0, rc
        return out, route, rw

    def vq_matvec(self, L, expert, kind, x, M):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(M, np.float32)
        assert self.L.ref_vq_matvec(self.m, L, expert, kind, _p(x), _p(y)) == 0
        return y

    def expert_ffn(self, L, expert, x, H):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(H, np.float32)
        assert self.L.ref_expert_ffn(self.m, L, expert, _p(x), _p(y)) == 0
        return y

    def save_usage(self, path):
        assert self.L.ref_save_usage(self.m, os.fsencode(path)) == 0

    def record_check(self, L, expert, rec, verify):
        """The reference's record_check on `rec` (uint8, the bank's record
        stride) as a record of (L, expert): 0 OK, 2 E_HEADER, 3 E_CRC."""
        rec = np.ascontiguousarray(rec, np.uint8)
        return self.L.ref_record_check(self.m, L, expert, _p(rec), int(verify))

    def n_books(self):
        return self.L.ref_n_books(self.m)

    def build_lut(self, L, kind, x, n_out):
        x = np.ascontiguousarray(x, np.float32)
        lut = np.empty(n_out, np.float32)
        self.L.ref_build_lut(self.m, L, kind, _p(x), x.shape[0], _p(lut))
        return lut


def ecache_replay(ids, n_slots):
    """The compiled reference's expert cache (oracle/_ref, src/ecache.c) on a
    routing trace ids [tokens][layers][K], one get per id in order (read-ahead
    and lookahead off): (hits, misses, evictions, records read)."""
    if not os.path.exists(REF_LIB):
        raise RuntimeError(f"{REF_LIB} is not built")
    L = C.CDLL(REF_LIB)
    L.ref_ecache_replay.restype = C.c_int
    L.ref_ecache_replay.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p]
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.zeros(4, np.uint64)
    n_tok, n_layers, K = ids.shape
    assert L.ref_ecache_replay(_p(ids), n_tok, n_layers, K, n_slots, _p(out)) == 0
    return tuple(int(v) for v in out)


def record_check(rec, layer, expert, fmt, stages, n_books, expert_m, verify):
    """or_record_check: the oracle's restatement of record_check
    (src/model.c:1698-1745) on a record of len(rec) bytes. fmt names the
    container's format (its index width); expert_m = rows of gate, up, down."""
    rec = np.ascontiguousarray(rec, np.uint8)
    bits = {"VQ3R": 8, "VQ2R": 8, "VQ4P": 6, "VQ12": 12}[fmt]
    m = np.ascontiguousarray(expert_m, np.int32)
    return lib().or_record_check(_p(rec), rec.size, layer, expert, bits, stages, n_books, _p(m), int(verify))


def kda_forward(q, k, v, g, beta, S):
    """T steps of or_kda_step: q, k, g [T][H][K], v [T][H][V], beta [T][H],
    S [H][K][V] (not modified). Returns (S after, o [T][H][V])."""
    T, H, K = q.shape
    V = v.shape[2]
    S = np.ascontiguousarray(S, np.float32).copy()
    o = np.empty((T, H, V), np.float32)
    for t in range(T):
        a = [np.ascontiguousarray(z[t], np.float32) for z in (q, k, v, g, beta)]
        lib().or_kda_step(H, K, V, *(_p(z) for z in a), _p(S), _p(o[t]))
    return S, o
