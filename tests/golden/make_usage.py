#!/usr/bin/env python3
"""Writes tests/golden/usage_vq3r.waste: a usage file written by the compiled
reference's own waste_model_save_usage (oracle/_ref) after decoding tokens
through a synthetic container with a small expert cache, so that the hit
counts differ between records. Run where the reference sources are built;
the file is data (the reference's usage format) and travels without them.
"""
import os
import shutil
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import container as ct  # noqa: E402
from oracle import pyoracle as po  # noqa: E402

SPEC = ct.Spec(hidden=128, inter=64, experts=16, top_k=3, layers=2, fmt="VQ3R", seed=211, bias=False)


def main():
    model = ct.build(SPEC)
    d = tempfile.mkdtemp(prefix="usage_")
    ct.write(model, d)
    ref = po.Ref(d, cache_bytes=12 * model.rec_bytes)           # 12 of the 32 records
    rng = np.random.default_rng(5)
    for t in range(40):
        x = rng.normal(size=SPEC.hidden).astype(np.float32)
        for L in range(SPEC.layers):
            ref.moe_layer(L, x, SPEC.experts, SPEC.top_k, SPEC.hidden)
    out = os.path.join(HERE, "usage_vq3r.waste")
    ref.save_usage(out)
    ref.close()
    shutil.rmtree(d)
    print(f"{out}: {os.path.getsize(out)} bytes")


if __name__ == "__main__":
    main()
