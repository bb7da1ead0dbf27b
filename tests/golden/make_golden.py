#!/usr/bin/env python3
"""Writes tests/golden/*.npz: inputs and outputs of the compiled reference
(oracle/_ref, built from the reference's own sources by oracle/Makefile) on
the synthetic containers of specs.py. Run in a container that has the
reference sources; the fixtures are data and travel without it.

Per spec: for every layer, moe_layer on 4 tokens (output, selection, router
logits, sigmoid scores), moe_chunk on 6 tokens (output, route, weights),
vq_matvec of every kind of expert 1, and the gate LUT of one input.
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import container as ct  # noqa: E402
from oracle import pyoracle as po  # noqa: E402
from specs import SPECS  # noqa: E402


def main():
    for name, spec in SPECS.items():
        model = ct.build(spec)
        d = tempfile.mkdtemp(prefix=f"golden_{name}_")
        ct.write(model, d)
        ref = po.Ref(d)
        rng = np.random.default_rng(1000 + spec.seed)
        H, I, E, K = spec.hidden, spec.inter, spec.experts, spec.top_k
        Hx = spec.latent or H                # the experts' width
        S, EN = ct.FMT_STAGES[spec.fmt], ct.FMT_ENTRIES[spec.fmt]
        out = {"digest": np.frombuffer(ct.digest(model).encode(), np.uint8), "backend": np.frombuffer(ref.backend().encode(), np.uint8)}
        for L in range(spec.layers):
            X = rng.normal(size=(4, H)).astype(np.float32)
            outs, idxs, lgs, scs = [], [], [], []
            for t in range(4):
                o, i, lg, sc = ref.moe_layer(L, X[t], E, K, H)
                outs.append(o); idxs.append(i); lgs.append(lg); scs.append(sc)
            out[f"L{L}_x"] = X
            out[f"L{L}_out"] = np.stack(outs)
            out[f"L{L}_idx"] = np.stack(idxs)
            out[f"L{L}_logits"] = np.stack(lgs)
            out[f"L{L}_scores"] = np.stack(scs)
            Xc = rng.normal(size=(6, H)).astype(np.float32)
            co, cr, cw = ref.moe_chunk(L, Xc, K, H)
            out[f"L{L}_chunk_x"] = Xc
            out[f"L{L}_chunk_out"] = co
            out[f"L{L}_chunk_route"] = cr
            out[f"L{L}_chunk_w"] = cw
            for kind in range(3):
                M, N = (I, Hx) if kind < 2 else (Hx, I)
                x = rng.normal(size=N).astype(np.float32)
                out[f"L{L}_mv{kind}_x"] = x
                out[f"L{L}_mv{kind}_y"] = ref.vq_matvec(L, 1, kind, x, M)
            x = rng.normal(size=Hx).astype(np.float32)
            out[f"L{L}_lut_x"] = x
            out[f"L{L}_lut"] = ref.build_lut(L, 0, x, (Hx // 8) * S * EN)
        ref.close()
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **out)
        print(f"{name}: {os.path.getsize(path)} bytes, backend {ref.backend() if False else out['backend'].tobytes().decode()}")


if __name__ == "__main__":
    main()
