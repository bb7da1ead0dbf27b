"""ctypes binding of libwarp_hip.so (include/warp_hip.h).

This is the host-side mirror of the reference's MoE interface: a `Context`
holds what waste_model_load keeps for the MoE layers (codebooks, routers,
shared experts, the expert cache) and exposes moe_layer / moe_chunk and the
finer kernels. Device buffers are passed as integer addresses (for example
torch.Tensor.data_ptr()); nothing here computes on the CPU, and every call
raises if the shared library is missing or the device call fails.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libwarp_hip.so")

VQ3R, VQ2R, VQ4P, VQ12 = 4, 5, 8, 9
FMT = {"VQ3R": VQ3R, "VQ2R": VQ2R, "VQ4P": VQ4P, "VQ12": VQ12}
ROUTE_SIGMOID, ROUTE_SOFTMAX = 0, 1
ERRORS = {-1: "E_ARG", -2: "E_DEVICE", -3: "E_NOMEM", -4: "E_READ", -5: "E_HEADER",
          -6: "E_CRC", -7: "E_NOSLOT", -8: "E_MISSING", -9: "E_BOOKS"}
E_ARG, E_DEVICE, E_NOMEM, E_READ, E_HEADER, E_CRC, E_NOSLOT, E_MISSING, E_BOOKS = range(-1, -10, -1)

_lib = None


class WarpHipError(RuntimeError):
    def __init__(self, code, msg, layer=-1, expert=-1):
        super().__init__(f"{ERRORS.get(code, code)}: {msg} (layer {layer}, expert {expert})")
        self.code, self.layer, self.expert = code, layer, expert


class Cfg(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("inter", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
        ("n_layers", C.c_int), ("fmt", C.c_int), ("renorm", C.c_int), ("routed_scale", C.c_float),
        ("router_act", C.c_int), ("router_strict", C.c_int), ("act_situ", C.c_int),
        ("situ_beta", C.c_float), ("situ_linear_beta", C.c_float), ("max_tokens", C.c_int),
        ("rec_bytes", C.c_size_t), ("cache_bytes", C.c_size_t), ("verify", C.c_int),
        ("lookahead", C.c_int), ("device", C.c_int), ("latent", C.c_int), ("latent_norm", C.c_int),
        ("norm_eps", C.c_float), ("prefill_fp16", C.c_int), ("n_books", C.c_int), ("router_fast", C.c_int),
    ]


class RouteStats(C.Structure):
    _fields_ = [("certified", C.c_uint64), ("recomputed", C.c_uint64), ("rows", C.c_uint64)]


class CacheStats(C.Structure):
    _fields_ = [("hits", C.c_uint64), ("misses", C.c_uint64), ("bytes_read", C.c_uint64),
                ("evictions", C.c_uint64), ("prefetched", C.c_uint64), ("spec_issued", C.c_uint64),
                ("n_slots", C.c_int), ("resident", C.c_int)]


FETCH_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_uint8))
FETCH_HOST_FN = C.CFUNCTYPE(C.c_void_p, C.c_void_p, C.c_int, C.c_int)


class TrunkTensor(C.Structure):
    """warp_trunk_tensor: a waste_tensor's F32 rows or quantised rows."""
    _fields_ = [("data", C.c_void_p), ("q", C.c_void_p), ("qs", C.c_void_p), ("group", C.c_int),
                ("bits", C.c_int), ("rowbytes", C.c_size_t)]


class MoeArgs(C.Structure):
    """warp_moe_args: one MoE layer of the engine's model and one call."""
    _fields_ = [
        ("model", C.c_void_p), ("layer", C.c_int), ("n_layers", C.c_int),
        ("hidden", C.c_int), ("moe_inter", C.c_int), ("n_experts", C.c_int), ("top_k", C.c_int),
        ("latent_dim", C.c_int), ("latent_norm", C.c_int), ("norm_eps", C.c_float), ("renorm", C.c_int),
        ("routed_scale", C.c_float), ("act_situ", C.c_int), ("situ_beta", C.c_float),
        ("situ_linear_beta", C.c_float), ("index_bits", C.c_int), ("stages", C.c_int), ("cb_entries", C.c_int),
        ("vec_dim", C.c_int), ("codebooks", C.c_void_p), ("n_books", C.c_int), ("cb_base", C.c_int),
        ("router", TrunkTensor), ("bias", C.c_void_p), ("shared", TrunkTensor * 3), ("inter_shared", C.c_int),
        ("latent", TrunkTensor * 2), ("latent_norm_w", C.c_void_p), ("rec_bytes", C.c_size_t),
        ("cache_bytes", C.c_size_t), ("verify", C.c_int), ("lookahead", C.c_int), ("fetch", FETCH_FN),
        ("fetch_user", C.c_void_p), ("n_tokens", C.c_int), ("x", C.c_void_p), ("out", C.c_void_p),
        ("route", C.c_void_p), ("rw", C.c_void_p),
    ]


MOE_SLOT = C.CFUNCTYPE(C.c_int, C.POINTER(MoeArgs))


class MoeKernels(C.Structure):
    """waste_moe_kernels: the MoE slots' table."""
    _fields_ = [("moe_ffn_decode", MOE_SLOT), ("moe_ffn_batch", MOE_SLOT), ("on_device", C.c_int)]

# name -> (restype, argtypes); also the list of symbols the header declares
SIGNATURES = {
    "waste_register_hip": (C.c_char_p, [C.c_void_p]),
    "waste_hip_release_host_buffers": (None, []),
    "waste_register_hip_moe": (C.c_char_p, [C.c_void_p]),
    "warp_hip_moe_table_stats": (None, [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "warp_hip_table_stats": (None, [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "warp_hip_kda_stats": (None, [C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "warp_hip_kda_forward": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "warp_hip_open": (C.c_int, [C.POINTER(Cfg), C.POINTER(C.c_void_p)]),
    "warp_hip_close": (None, [C.c_void_p]),
    "warp_hip_error": (C.c_char_p, [C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "warp_hip_stream": (C.c_void_p, [C.c_void_p]),
    "warp_hip_set_codebooks": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "warp_hip_set_router": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    "warp_hip_set_router_q": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                        C.c_size_t, C.c_void_p]),
    "warp_hip_set_shared": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p * 3,
                                      C.c_void_p * 3, C.c_size_t * 3]),
    "warp_hip_set_latent": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_size_t,
                                      C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "warp_hip_set_fetch": (C.c_int, [C.c_void_p, FETCH_FN, C.c_void_p]),
    "warp_hip_set_fetch_host": (C.c_int, [C.c_void_p, FETCH_HOST_FN, C.c_void_p]),
    "warp_hip_host_alloc": (C.c_void_p, [C.c_void_p, C.c_size_t]),
    "warp_hip_host_free": (None, [C.c_void_p, C.c_void_p]),
    "warp_hip_put_expert": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "warp_hip_prefetch": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int]),
    "warp_hip_get_cache_stats": (None, [C.c_void_p, C.POINTER(CacheStats)]),
    "warp_hip_get_route_stats": (C.c_int, [C.c_void_p, C.POINTER(RouteStats)]),
    "warp_hip_router_cert": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    "warp_hip_moe_decode": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p]),
    "warp_hip_moe_decode_host": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]),
    "warp_hip_expert_ffn": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "warp_hip_moe_chunk": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                     C.c_void_p, C.c_void_p]),
    "warp_hip_moe_chunk_host": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                          C.c_void_p]),
    "warp_hip_vq_matvec": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]),
    "warp_hip_decode_weights": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "warp_hip_router_logits": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]),
    "warp_hip_route": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    "warp_hip_mvq": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p,
                               C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "warp_hip_fill_random": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_uint64]),
    "warp_hip_crc32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(C.c_uint32)]),
    "warp_hip_save_usage": (C.c_int, [C.c_void_p, C.c_char_p, C.c_uint64]),
    "warp_hip_warm": (C.c_int, [C.c_void_p, C.c_char_p]),
    "warp_hip_resident": (C.c_void_p, [C.c_void_p, C.c_int, C.c_int]),
    "warp_hip_put_expert_dev": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "warp_hip_put_expert_synth": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_uint64, C.c_void_p]),
    "warp_hip_set_matvec_path": (C.c_int, [C.c_void_p, C.c_int]),
    "warp_hip_set_router_fast": (C.c_int, [C.c_void_p, C.c_int]),
    "warp_hip_set_cert_polls": (C.c_int, [C.c_void_p, C.c_uint]),
    "warp_hip_matvec_kernel": (C.c_char_p, [C.c_void_p, C.c_int, C.c_int]),
    "warp_hip_set_timing": (C.c_int, [C.c_void_p, C.c_int]),
    "warp_hip_get_timing": (C.c_int, [C.c_void_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    "warp_hip_sync": (C.c_int, [C.c_void_p]),
    "warp_hip_vq_encode": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                                     C.c_int]),
    "warp_hip_vq_encode16": (C.c_int, [C.c_void_p, C.c_long, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "warp_hip_vq_encode_dev": (C.c_int, [C.c_void_p, C.c_long, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                         C.c_void_p, C.c_void_p]),
    "warp_hip_vq_lloyd": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "warp_hip_vq_encode_dev_noalloc": (C.c_int, [C.c_void_p, C.c_long, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                                 C.c_void_p]),
}


def lib():
    """The loaded library. Raises if it has not been built: there is no other
    implementation to fall back to."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run warp_amd.build.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _addr(x):
    """Address of a device buffer (torch tensor or int) or a numpy array."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if hasattr(x, "ctypes"):
        return x.ctypes.data
    raise TypeError(type(x))


class Context:
    def __init__(self, *, hidden, inter, n_experts, top_k, n_layers, fmt, renorm=True,
                 routed_scale=1.0, router_act=ROUTE_SIGMOID, router_strict=False, act_situ=False,
                 situ_beta=1.0, situ_linear_beta=0.0, max_tokens=1, rec_bytes, cache_bytes,
                 verify=False, lookahead=0, device=0, latent=0, latent_norm=True, norm_eps=1e-5,
                 prefill_fp16=False, n_books=0, router_fast=False):
        self.cfg = Cfg(hidden, inter, n_experts, top_k, n_layers, FMT.get(fmt, fmt), int(renorm),
                       routed_scale, router_act, int(router_strict), int(act_situ), situ_beta,
                       situ_linear_beta, max_tokens, rec_bytes, cache_bytes, int(verify), lookahead, device,
                       latent, int(latent_norm), norm_eps, int(prefill_fp16), n_books, int(router_fast))
        self.h = C.c_void_p()
        self._keep = []
        rc = lib().warp_hip_open(C.byref(self.cfg), C.byref(self.h))
        if rc:
            raise WarpHipError(rc, "warp_hip_open failed (see stderr)")

    # -- plumbing
    def _check(self, rc):
        if rc:
            lay, exp = C.c_int(), C.c_int()
            msg = lib().warp_hip_error(self.h, C.byref(lay), C.byref(exp)).decode()
            raise WarpHipError(rc, msg, lay.value, exp.value)

    def close(self):
        if self.h:
            lib().warp_hip_close(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        return lib().warp_hip_stream(self.h)

    def sync(self):
        self._check(lib().warp_hip_sync(self.h))

    # -- weights
    def set_codebooks(self, layer, cb_base, books_u16):
        self._check(lib().warp_hip_set_codebooks(self.h, layer, cb_base, _addr(books_u16)))

    def set_router(self, layer, w_f32, bias=None):
        self._check(lib().warp_hip_set_router(self.h, layer, _addr(w_f32), _addr(bias)))

    def set_router_q(self, layer, bits, group, q, scales, rowbytes, bias=None):
        self._check(lib().warp_hip_set_router_q(self.h, layer, bits, group, _addr(q), _addr(scales), rowbytes,
                                                _addr(bias)))

    def set_shared(self, layer, bits, group, inter_shared, qs, ss, rowbytes):
        qa = (C.c_void_p * 3)(*[_addr(q) for q in qs])
        sa = (C.c_void_p * 3)(*[_addr(s) for s in ss])
        ra = (C.c_size_t * 3)(*rowbytes)
        self._check(lib().warp_hip_set_shared(self.h, layer, bits, group, inter_shared, qa, sa, ra))

    def set_latent(self, layer, bits, group, down, up, norm_w=None):
        """down/up: (payload, scales, rowbytes) of routed_expert_down_proj
        [latent][H] and routed_expert_up_proj [H][latent]."""
        self._check(lib().warp_hip_set_latent(self.h, layer, bits, group, _addr(down[0]), _addr(down[1]), down[2],
                                              _addr(up[0]), _addr(up[1]), up[2], _addr(norm_w)))

    # -- experts
    def put_expert(self, layer, expert, rec):
        self._check(lib().warp_hip_put_expert(self.h, layer, expert, _addr(rec)))

    def put_expert_dev(self, layer, expert, rec_dev):
        self._check(lib().warp_hip_put_expert_dev(self.h, layer, expert, _addr(rec_dev)))

    def set_fetch(self, fn):
        """fn(layer, expert) -> bytes of one record, or None on failure. A
        record of any length other than rec_bytes is a failed fetch (the
        staging slot holds exactly one record)."""
        rec_bytes = self.cfg.rec_bytes

        def cb(_user, layer, expert, dst):
            try:
                data = fn(layer, expert)
                if data is None or len(data) != rec_bytes:
                    return -1
                C.memmove(dst, data, rec_bytes)
                return 0
            except Exception:
                return -1
        self._fetch_cb = FETCH_FN(cb)
        self._check(lib().warp_hip_set_fetch(self.h, self._fetch_cb, None))

    def set_fetch_host(self, fn):
        """fn(layer, expert) -> address (int) of the record in pinned host
        memory from host_alloc, or 0/None when it cannot; the miss copies it
        to HBM from there."""
        def cb(_user, layer, expert):
            try:
                return fn(layer, expert) or None
            except Exception:
                return None
        self._fetch_host_cb = FETCH_HOST_FN(cb)
        self._check(lib().warp_hip_set_fetch_host(self.h, self._fetch_host_cb, None))

    def host_alloc(self, nbytes):
        """Pinned host memory as a uint8 numpy array (freed with host_free)."""
        import numpy as np
        p = lib().warp_hip_host_alloc(self.h, nbytes)
        if not p:
            self._check(E_NOMEM)
        return np.ctypeslib.as_array((C.c_uint8 * nbytes).from_address(p))

    def host_free(self, arr):
        """Free host_alloc memory: after every copy from it has finished
        (a synchronising call, or close)."""
        lib().warp_hip_host_free(self.h, arr.ctypes.data)

    def prefetch(self, layer, ids):
        import numpy as np
        a = np.ascontiguousarray(ids, dtype=np.int32)
        self._check(lib().warp_hip_prefetch(self.h, layer, a.ctypes.data, len(a)))

    def resident(self, layer, expert):
        return lib().warp_hip_resident(self.h, layer, expert)

    def router_cert(self, layer, x_dev, out_dev):
        """The certified router's [4][E] arrays for one token: point scores,
        point biased scores, lower and upper bounds of the biased score."""
        self._check(lib().warp_hip_router_cert(self.h, layer, _addr(x_dev), _addr(out_dev)))

    def route_stats(self):
        """Certified selection's counters: decode routings certified, those
        that recomputed rows, and the rows recomputed."""
        st = RouteStats()
        self._check(lib().warp_hip_get_route_stats(self.h, C.byref(st)))
        return {k: getattr(st, k) for k, _ in RouteStats._fields_}

    def cache_stats(self):
        st = CacheStats()
        lib().warp_hip_get_cache_stats(self.h, C.byref(st))
        return {k: getattr(st, k) for k, _ in CacheStats._fields_}

    # -- the layer
    def moe_decode(self, layer, x_dev, out_dev, resid_dev=None, want_route=False):
        import numpy as np
        K = self.cfg.top_k
        idx = np.empty(K, np.int32) if want_route else None
        w = np.empty(K, np.float32) if want_route else None
        self._check(lib().warp_hip_moe_decode(self.h, layer, _addr(x_dev), _addr(out_dev), _addr(resid_dev),
                                              _addr(idx), _addr(w)))
        return (idx, w) if want_route else None

    def expert_ffn(self, layer, expert, x_dev, out_dev):
        """One resident expert's FFN on one token (no routing), queued."""
        self._check(lib().warp_hip_expert_ffn(self.h, layer, expert, _addr(x_dev), _addr(out_dev)))

    def moe_decode_host(self, layer, x):
        import numpy as np
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(self.cfg.hidden, np.float32)
        routed = np.empty(self.cfg.top_k, np.int32)
        self._check(lib().warp_hip_moe_decode_host(self.h, layer, x.ctypes.data, out.ctypes.data,
                                                   routed.ctypes.data))
        return out, routed

    def moe_chunk(self, layer, X_dev, out_dev, T, want_route=False, resid_dev=None):
        import numpy as np
        K = self.cfg.top_k
        route = np.empty((T, K), np.int32) if want_route else None
        rw = np.empty((T, K), np.float32) if want_route else None
        self._check(lib().warp_hip_moe_chunk(self.h, layer, _addr(X_dev), _addr(out_dev), _addr(resid_dev), T,
                                             _addr(route), _addr(rw)))
        return (route, rw) if want_route else None

    def moe_chunk_host(self, layer, X):
        import numpy as np
        X = np.ascontiguousarray(X, np.float32)
        T = X.shape[0]
        out = np.empty((T, self.cfg.hidden), np.float32)
        route = np.empty((T, self.cfg.top_k), np.int32)
        rw = np.empty((T, self.cfg.top_k), np.float32)
        self._check(lib().warp_hip_moe_chunk_host(self.h, layer, X.ctypes.data, out.ctypes.data, T,
                                                  route.ctypes.data, rw.ctypes.data))
        return out, route, rw

    # -- finer kernels
    def vq_matvec(self, layer, kind, rec_dev, x_dev, y_dev):
        self._check(lib().warp_hip_vq_matvec(self.h, layer, kind, _addr(rec_dev), _addr(x_dev), _addr(y_dev)))

    def decode_weights(self, layer, kind, rec_dev, W_dev):
        self._check(lib().warp_hip_decode_weights(self.h, layer, kind, _addr(rec_dev), _addr(W_dev)))

    def router_logits(self, layer, x_dev, T, logits_dev):
        self._check(lib().warp_hip_router_logits(self.h, layer, _addr(x_dev), T, _addr(logits_dev)))

    def route(self, layer, logits_dev, T, idx_dev, w_dev):
        self._check(lib().warp_hip_route(self.h, layer, _addr(logits_dev), T, _addr(idx_dev), _addr(w_dev)))

    def mvq(self, bits, group, q_dev, s_dev, rowbytes, x_dev, M, N, T, y_dev):
        self._check(lib().warp_hip_mvq(self.h, bits, group, _addr(q_dev), _addr(s_dev), rowbytes, _addr(x_dev),
                                       M, N, T, _addr(y_dev)))

    def put_expert_synth(self, layer, expert, seed, scales_u16):
        self._check(lib().warp_hip_put_expert_synth(self.h, layer, expert, seed, _addr(scales_u16)))

    def set_matvec_path(self, path):
        """"auto" (the LUT kernel for decode where it applies, the gather
        kernel for small shapes), "mfma", "fused" (the LUT kernel's gate/up,
        down and combine in one launch per layer where it routes the token
        itself) or "gather" (decode-then-dot with codebook gathers)."""
        code = {"auto": 0, "mfma": 1, "fused": 2, "gather": 3}[path]
        self._check(lib().warp_hip_set_matvec_path(self.h, code))

    def set_router_fast(self, fast):
        """True: decode from the fast logits' picks uncertified; False: certify."""
        self._check(lib().warp_hip_set_router_fast(self.h, int(bool(fast))))
        self.cfg.router_fast = int(bool(fast))

    def set_cert_polls(self, polls):
        """The certifying router's poll limit for its rows (0: the default);
        a launch that reaches it gives up and the next sync reports E_DEVICE."""
        self._check(lib().warp_hip_set_cert_polls(self.h, int(polls)))

    def matvec_kernel(self, layer, expert_ffn=False):
        """The expert matvec kernel a decode of `layer` runs on the current path."""
        return lib().warp_hip_matvec_kernel(self.h, layer, 1 if expert_ffn else self.cfg.top_k).decode()

    def set_timing(self, on):
        self._check(lib().warp_hip_set_timing(self.h, int(on)))

    def get_timing(self):
        ms = (C.c_double * 4)()
        n = (C.c_uint64 * 4)()
        self._check(lib().warp_hip_get_timing(self.h, ms, n))
        return list(ms), list(n)

    def crc32(self, dev, nbytes):
        """zlib's crc32 of nbytes of device memory, computed on the device."""
        out = C.c_uint32()
        self._check(lib().warp_hip_crc32(self.h, _addr(dev), nbytes, C.byref(out)))
        return out.value

    def save_usage(self, path, tokens=0):
        self._check(lib().warp_hip_save_usage(self.h, os.fsencode(path), tokens))

    def warm(self, path):
        """Fill the cache with the hottest records of a usage file; returns
        how many were loaded."""
        n = lib().warp_hip_warm(self.h, os.fsencode(path))
        if n < 0:
            self._check(n)
        return n

    def fill_random(self, dev, nbytes, seed):
        self._check(lib().warp_hip_fill_random(self.h, _addr(dev), nbytes, seed))


def _check_rc(rc, what):
    if rc < 0:
        raise WarpHipError(rc, what)
    return rc


def vq_encode(X, books):
    """waste_vq_encode on the device: X [n][8] f32, books [stages][entries][8]
    f32 -> codes [n][stages] (uint8 for up to 256 entries, else uint16)."""
    import numpy as np
    X = np.ascontiguousarray(X, np.float32)
    books = np.ascontiguousarray(books, np.float32)
    n, (S, E, D) = X.shape[0], books.shape
    if E <= 256:
        out = np.empty((n, S), np.uint8)
        _check_rc(lib().warp_hip_vq_encode(X.ctypes.data, n, books.ctypes.data, S, E, D, out.ctypes.data, 0),
                  "vq_encode")
    else:
        out = np.empty((n, S), np.uint16)
        _check_rc(lib().warp_hip_vq_encode16(X.ctypes.data, n, books.ctypes.data, S, E, D, out.ctypes.data),
                  "vq_encode16")
    return out


def vq_lloyd(X, C):
    """One waste_vq_lloyd iteration on the device; C [entries][8] is updated
    in place. Returns the number of non-empty clusters."""
    import numpy as np
    X = np.ascontiguousarray(X, np.float32)
    assert C.dtype == np.float32 and C.flags.c_contiguous
    return _check_rc(lib().warp_hip_vq_lloyd(X.ctypes.data, X.shape[0], C.ctypes.data, C.shape[0], C.shape[1], 0),
                     "vq_lloyd")


def load_container_model(ctx: Context, model, layers=None, records=True):
    """Upload one tests/golden/container.Model (or anything with the same
    attributes) into a context: codebooks, routers, latent projections,
    shared experts and (unless records is False, for a context that fetches
    them on a miss) the expert records."""
    import numpy as np
    spec = model.spec
    S = {"VQ3R": 3, "VQ2R": 2, "VQ4P": 4, "VQ12": 2}[spec.fmt]
    layers = range(spec.layers) if layers is None else layers
    for L in layers:
        lay = model.layers[L]
        base = L * 3 * S
        books = np.ascontiguousarray(model.books_raw[base:base + 3 * S])
        ctx.set_codebooks(L, base, books)
        if lay.router_q is None:
            ctx.set_router(L, np.ascontiguousarray(lay.router, np.float32), lay.bias)
        else:
            pl, sc, rb, bits, group = lay.router_q
            ctx.set_router_q(L, bits, group, np.ascontiguousarray(pl), np.ascontiguousarray(sc), rb, lay.bias)
        if getattr(lay, "latent", None) is not None:
            dq, uq, nw = lay.latent
            ctx.set_latent(L, dq[3], dq[4], (np.ascontiguousarray(dq[0]), np.ascontiguousarray(dq[1]), dq[2]),
                           (np.ascontiguousarray(uq[0]), np.ascontiguousarray(uq[1]), uq[2]), nw)
        if lay.shared:
            ctx.set_shared(L, spec.shared_bits, spec.shared_group, spec.inter * spec.n_shared,
                           [np.ascontiguousarray(s[0]) for s in lay.shared],
                           [np.ascontiguousarray(s[1]) for s in lay.shared], [s[2] for s in lay.shared])
        for e, rec in enumerate(lay.records if records else ()):
            if rec is not None:                  # experts without a record stay out of the cache
                ctx.put_expert(L, e, np.frombuffer(rec, np.uint8))
