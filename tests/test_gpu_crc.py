"""zlib's crc32 on the device, the payload checksum of records entering the
HBM cache (cfg.verify), and the learned hotlist (usage file) warm.

- warp_hip_crc32 against the reference's own known answers for its
  waste_crc32 (tests/test_container.c:36-66 in the reference: zlib's values
  for short strings and for a 64 KiB pattern at several offsets and
  lengths), and against Python's zlib on random buffers of lengths around
  the kernels' 64-byte and 64 KiB pieces, up to a K3-size record, from
  unaligned starts.
- With verify, a record whose payload does not match its header's checksum
  is refused on every path that fills the cache: the fetch callback's
  staging copy, the pinned host tier, put_expert, put_expert_dev; the call
  fails with E_CRC naming the record, the record does not stay resident,
  and a good copy of it is taken afterwards. A refused speculative fill
  (lookahead) is reported by the next call that waits.
- warp_hip_warm reads a usage file written by the compiled reference's own
  waste_model_save_usage (tests/golden/usage_vq3r.waste, from
  tests/golden/make_usage.py) and fills the cache with its hottest records
  in the reference's order (hits descending, then layer and expert,
  src/ecache.c:749-760); warp_hip_save_usage writes the same format back.
"""
import os
import struct
import zlib

import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def small():
    import warp_amd
    spec = ct.Spec(hidden=256, inter=128, experts=16, top_k=3, layers=2, fmt="VQ12", seed=91, **BALANCED)
    model = ct.build(spec)
    ctx = open_ctx(model)
    warp_amd.load_container_model(ctx, model)
    yield model, ctx
    ctx.close()


def test_device_crc32_known_answers(small):
    model, ctx = small
    for s, want in ((b"a", 0xE8B7BE43), (b"123456789", 0xCBF43926),
                    (b"The quick brown fox jumps over the lazy dog", 0x414FA339)):
        assert ctx.crc32(dev(np.frombuffer(s, np.uint8)), len(s)) == want, s
    assert ctx.crc32(0, 0) == 0
    i = np.arange(65536, dtype=np.uint64)
    pat = ((i * 31 + (i >> 11)) & 0xFF).astype(np.uint8)
    pd = dev(pat)
    for off, n, want in ((0, 65536, 0x857C6B4F), (0, 3071, 0xE08F605E), (0, 3073, 0x331C420A),
                         (3, 40001, 0x5BBC9F51), (7, 65529, 0xB1F5AE9A)):
        assert ctx.crc32(pd.ptr + off, n) == want, (off, n)
    rng = np.random.default_rng(3)
    buf = rng.integers(0, 256, size=16_537_600 + 4096, dtype=np.uint8)
    bd = dev(buf)
    for off, n in ((0, 1), (1, 63), (0, 64), (5, 65), (0, 4095), (3, 65535), (0, 65536), (1, 65537),
                   (7, 1_000_003), (48, 16_537_600), (0, 16_537_600 + 4096)):
        assert ctx.crc32(bd.ptr + off, n) == zlib.crc32(buf[off:off + n].tobytes()), (off, n)
    log("device crc32: the reference's known answers and zlib on 1 B .. 16.5 MB, unaligned starts")


SPEC = dict(hidden=256, inter=128, experts=16, top_k=3, layers=2, fmt="VQ12", seed=93, **BALANCED)


def verify_ctx(model, slots, lookahead=0):
    ctx = open_ctx(model, max_tokens=4, cache_slots=slots, verify=True, lookahead=lookahead)
    S = ct.FMT_STAGES[model.spec.fmt]
    for L in range(model.spec.layers):
        lay = model.layers[L]
        ctx.set_codebooks(L, L * 3 * S, np.ascontiguousarray(model.books_raw[L * 3 * S:(L + 1) * 3 * S]))
        ctx.set_router(L, np.ascontiguousarray(lay.router, np.float32), lay.bias)
        s = model.spec
        ctx.set_shared(L, s.shared_bits, s.shared_group, s.inter, [np.ascontiguousarray(q[0]) for q in lay.shared],
                       [np.ascontiguousarray(q[1]) for q in lay.shared], [q[2] for q in lay.shared])
    return ctx


def corrupt(rec, at=5000):
    b = bytearray(rec)
    b[at] ^= 0x10
    return bytes(b)


@pytest.mark.parametrize("mode", ["copy", "host"])
def test_verify_refuses_a_corrupt_fetch(mode):
    import warp_amd
    model = ct.build(ct.Spec(**SPEC))
    x = np.random.default_rng(4).normal(size=SPEC["hidden"]).astype(np.float32)
    idx = np.asarray(po.LayerView(model, 0).moe_layer(x)[1])
    bad_e = int(idx[1])                                   # the second pick's record is damaged
    recs = {(L, e): r for L in range(2) for e, r in enumerate(model.layers[L].records)}
    recs[(0, bad_e)] = corrupt(recs[(0, bad_e)])
    ctx = verify_ctx(model, slots=8)
    pool = None
    try:
        if mode == "copy":
            ctx.set_fetch(lambda L, e: recs.get((L, e)))
        else:
            keys = sorted(recs)
            pool = ctx.host_alloc(len(keys) * model.rec_bytes)
            where = {}
            for i, k in enumerate(keys):
                pool[i * model.rec_bytes:(i + 1) * model.rec_bytes] = np.frombuffer(recs[k], np.uint8)
                where[k] = pool.ctypes.data + i * model.rec_bytes
            ctx.set_fetch_host(lambda L, e: where.get((L, e)))
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.moe_decode(0, dev(x), empty(SPEC["hidden"]))
        assert ei.value.code == warp_amd.E_CRC and (ei.value.layer, ei.value.expert) == (0, bad_e), ei.value
        assert not ctx.resident(0, bad_e)
        for e in idx:
            if e != bad_e:
                assert ctx.resident(0, int(e))
        # the good copy is taken afterwards, and the layer computes
        good = model.layers[0].records[bad_e]
        ctx.put_expert(0, bad_e, np.frombuffer(good, np.uint8))
        out = empty(SPEC["hidden"])
        got_idx, _ = ctx.moe_decode(0, dev(x), out, want_route=True)
        assert np.array_equal(got_idx, idx) and np.isfinite(host(out)).all()
        log(f"verify ({mode} fetch): expert {bad_e} refused with E_CRC, not resident; its good copy taken after")
    finally:
        ctx.close()
        if pool is not None:
            ctx.host_free(pool)


def test_verify_on_put_paths_and_prefetch():
    import warp_amd
    model = ct.build(ct.Spec(**SPEC))
    ctx = verify_ctx(model, slots=32, lookahead=0)
    try:
        good = np.frombuffer(model.layers[1].records[4], np.uint8)
        bad = np.frombuffer(corrupt(model.layers[1].records[4], at=20000), np.uint8)
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.put_expert(1, 4, bad)
        assert ei.value.code == warp_amd.E_CRC and (ei.value.layer, ei.value.expert) == (1, 4)
        assert not ctx.resident(1, 4)
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.put_expert_dev(1, 4, dev(bad))
        assert ei.value.code == warp_amd.E_CRC and not ctx.resident(1, 4)
        ctx.put_expert_dev(1, 4, dev(good))
        assert ctx.resident(1, 4)
        # a speculative fill: reported by the next call that waits
        recs = {(L, e): r for L in range(2) for e, r in enumerate(model.layers[L].records)}
        recs[(1, 9)] = corrupt(recs[(1, 9)])
        ctx.set_fetch(lambda L, e: recs.get((L, e)))
        ctx.prefetch(1, [9, 10])
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.sync()
        assert ei.value.code == warp_amd.E_CRC and (ei.value.layer, ei.value.expert) == (1, 9)
        assert not ctx.resident(1, 9) and ctx.resident(1, 10)
        ctx.sync()                                        # reported once
        log("verify: put_expert, put_expert_dev and a prefetch refuse corrupt records (E_CRC)")
    finally:
        ctx.close()


USAGE_SPEC = dict(hidden=128, inter=64, experts=16, top_k=3, layers=2, fmt="VQ3R", seed=211, bias=False)


def read_usage(path):
    b = open(path, "rb").read()
    magic, version, tokens = struct.unpack("<IIQ", b[:16])
    ent = np.frombuffer(b[16:], dtype=[("layer", "<u2"), ("expert", "<u2"), ("hits", "<u4"), ("last", "<u4"),
                                       ("next", "<u4")])
    return magic, version, tokens, ent


@pytest.mark.parametrize("slots", [5, 20])
def test_warm_from_the_reference_usage_file(slots, tmp_path):
    import warp_amd
    model = ct.build(ct.Spec(**USAGE_SPEC))
    path = os.path.join(HERE, "usage_vq3r.waste")
    magic, version, tokens, ent = read_usage(path)
    assert magic == 0x47535557 and version == 1 and len(ent) == 12
    # the reference's warm order: hits descending, then layer, then expert
    order = sorted(ent.tolist(), key=lambda r: (-r[2], r[0], r[1]))
    want = order[:min(slots, len(order))]
    ctx = open_ctx(model, max_tokens=4, cache_slots=slots)
    try:
        S = ct.FMT_STAGES["VQ3R"]
        for L in range(2):
            ctx.set_codebooks(L, L * 3 * S, np.ascontiguousarray(model.books_raw[L * 3 * S:(L + 1) * 3 * S]))
            ctx.set_router(L, np.ascontiguousarray(model.layers[L].router, np.float32), model.layers[L].bias)
        recs = {(L, e): r for L in range(2) for e, r in enumerate(model.layers[L].records)}
        asked = []

        def fetch(L, e):
            asked.append((L, e))
            return recs.get((L, e))
        ctx.set_fetch(fetch)
        n = ctx.warm(path)
        assert n == len(want), (n, want)
        assert asked == [(r[0], r[1]) for r in want]       # fetched hottest first
        resident = {(L, e) for L in range(2) for e in range(16) if ctx.resident(L, e)}
        assert resident == {(r[0], r[1]) for r in want}
        st = ctx.cache_stats()
        assert st["misses"] == 0 and st["prefetched"] == n, st
        out = str(tmp_path / "usage.waste")
        ctx.save_usage(out, tokens=77)
        m2, v2, t2, e2 = read_usage(out)
        assert (m2, v2, t2) == (0x47535557, 1, 77)
        assert sorted((int(r[0]), int(r[1]), int(r[2])) for r in e2) == sorted((r[0], r[1], r[2]) for r in want)
        # stale entries (a layer or expert this context does not have) are
        # skipped; the one valid entry is loaded, evicting when the cache is
        # full, as the reference's warm takes a victim (src/ecache.c:796-800)
        stale = str(tmp_path / "stale.waste")
        with open(stale, "wb") as f:
            f.write(struct.pack("<IIQ", 0x47535557, 1, 0))
            f.write(struct.pack("<HHIII", 7, 3, 1000, 0, 0))
            f.write(struct.pack("<HHIII", 0, 99, 999, 0, 0))
            f.write(struct.pack("<HHIII", 1, 3, 1, 0, 0))
        assert not ctx.resident(1, 3)
        assert ctx.warm(stale) == 1 and ctx.resident(1, 3)
        with pytest.raises(warp_amd.WarpHipError):
            ctx.warm(str(tmp_path / "missing.waste"))
        log(f"warm ({slots} slots): {n} records from the reference's usage file in its order; save_usage round trip")
    finally:
        ctx.close()
