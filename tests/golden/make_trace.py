#!/usr/bin/env python3
"""Writes tests/golden/trace_kimi_300.npz: the reference's real routing trace
(its tests/trace_kimi_300.jsonl: 300 tokens x 26 MoE layers x top-8 of 256,
Kimi-Linear) as ids [300][26][8], and the compiled reference's expert cache
(oracle/_ref, src/ecache.c) replayed over it at several cache sizes: the
hits, misses, evictions and records read it counts with read-ahead and
lookahead off. Run in a container that has the reference sources; the
fixture is data and travels without them."""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import pyoracle as po  # noqa: E402

TRACE = "/root/reference/tests/trace_kimi_300.jsonl"
SLOTS = (64, 208, 512, 1024, 2048)


def main():
    rows = [json.loads(l) for l in open(TRACE)]
    ids = np.array([r["layers"] for r in rows], np.int16)
    assert ids.shape == (300, 26, 8)
    counts = np.array([po.ecache_replay(ids, n) for n in SLOTS], np.int64)
    np.savez_compressed(os.path.join(HERE, "trace_kimi_300.npz"), ids=ids, slots=np.array(SLOTS, np.int32),
                        ref_counts=counts)
    for n, c in zip(SLOTS, counts):
        print(f"slots {n:5d}: hits {c[0]} misses {c[1]} evictions {c[2]} hit rate {c[0] / (c[0] + c[1]):.4f}")


if __name__ == "__main__":
    main()
