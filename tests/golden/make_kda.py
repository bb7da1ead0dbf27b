#!/usr/bin/env python3
"""Writes tests/golden/kda.npz: inputs and outputs of the compiled reference's
waste_kda_step (oracle/_ref, src/kda.c:26-68) over a few steps and shapes.
Run where the reference sources are built; the fixture is data."""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import pyoracle as po  # noqa: E402

CASES = [(3, 2, 16, 16), (2, 3, 32, 48), (2, 2, 64, 128)]        # (T, H, K, V)


def main():
    L = C.CDLL(po.REF_LIB)
    vp, i = C.c_void_p, C.c_int
    L.waste_kda_step.argtypes = [i, i, i, vp, vp, vp, vp, vp, vp, vp, vp]
    L.waste_kda_step.restype = None
    out = {}
    rng = np.random.default_rng(17)
    for n, (T, H, K, V) in enumerate(CASES):
        q = rng.normal(size=(T, H, K)).astype(np.float32)
        k = rng.normal(size=(T, H, K)).astype(np.float32)
        v = rng.normal(size=(T, H, V)).astype(np.float32)
        g = -rng.uniform(0.0, 2.0, size=(T, H, K)).astype(np.float32)
        beta = rng.uniform(0.0, 1.0, size=(T, H)).astype(np.float32)
        S0 = (rng.normal(size=(H, K, V)) * 0.1).astype(np.float32)
        S = S0.copy()
        o = np.empty((T, H, V), np.float32)
        u = np.empty(V, np.float32)
        for t in range(T):
            a = [np.ascontiguousarray(z[t]) for z in (q, k, v, g, beta)]
            L.waste_kda_step(H, K, V, *(z.ctypes.data for z in a), S.ctypes.data, o[t].ctypes.data, u.ctypes.data)
        for name, arr in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta), ("S0", S0), ("S", S), ("o", o)):
            out[f"c{n}_{name}"] = arr
    path = os.path.join(HERE, "kda.npz")
    np.savez_compressed(path, **out)
    print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
