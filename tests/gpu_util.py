"""Shared helpers for the GPU parity tests: a context loaded from a synthetic
container, device buffers through the library's HIP runtime, and the
comparison metrics."""
import sys

import numpy as np

import container as ct
from oracle import pyoracle as po


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a):
    """A device copy of a numpy array (the library's own HIP runtime)."""
    from warp_amd.device import Buf
    return Buf.of(a)


def empty(shape, dtype=np.float32):
    from warp_amd.device import Buf
    return Buf.empty(shape, dtype)


def host(b):
    return b.numpy()


# Synthetic magnitudes for layer-level GPU tests: codebooks N(0, 0.3) (a
# normalised codebook's spread; with U(0.01, 0.05) row scales the decoded
# weights are ~1e-2) and shared-expert group scales of 1e-4..3e-4, so that
# the routed experts and the shared expert both show in a layer's output.
BALANCED = dict(book_std=0.3, shared_scale=(1e-4, 3e-4))


def routed_share(model, layer, x):
    """max|routed part| / max|layer output| for one token, from the oracle:
    the same layer with its shared expert taken out. A layer test is only
    sensitive to the routed path when this is not tiny."""
    import copy
    m = copy.copy(model)
    m.layers = list(model.layers)
    lay = copy.copy(model.layers[layer])
    lay.shared = []
    m.layers[layer] = lay
    full = po.LayerView(model, layer).moe_layer(x)[0]
    routed = po.LayerView(m, layer).moe_layer(x)[0]
    return float(np.max(np.abs(routed)) / max(np.max(np.abs(full)), 1e-30))


def rel_err(got, ref):
    """max|got - ref| / max|ref|, the tolerance metric the parity bar uses."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (den if den > 0 else 1.0))


def open_ctx(model, max_tokens=1, cache_slots=None, **kw):
    import warp_amd
    s = model.spec
    n = cache_slots if cache_slots is not None else s.layers * s.experts
    ctx = warp_amd.Context(hidden=s.hidden, inter=s.inter, n_experts=s.experts, top_k=s.top_k,
                           n_layers=s.layers, fmt=s.fmt, renorm=s.renorm, routed_scale=s.routed_scale,
                           act_situ=s.act == "situ", situ_beta=s.situ_beta, situ_linear_beta=s.situ_lbeta,
                           max_tokens=max_tokens, rec_bytes=model.rec_bytes,
                           cache_bytes=n * model.rec_bytes, latent=s.latent, latent_norm=s.latent_norm, **kw)
    return ctx
