"""Record verification against the reference's record_check, and the
records' own codebook ids.

- Every damaged header of tests/golden/recchk.npz (one per condition of
  src/model.c:1703-1738, from the compiled reference) goes through
  warp_hip_put_expert and through the fetch path (a prefetch), with the
  checksum off and on: the call is refused exactly where the reference
  refuses, with the code of the reference's status (E_HEADER for
  REC_E_HEADER, E_CRC for REC_E_CRC). The three cases marked `stricter`
  (increasing offsets whose index blocks are shorter than the shape) are
  refused here with E_HEADER where the reference accepts them, because the
  kernels index each block's whole shape.
- A record is decoded with its own codebook_id, as the reference does
  (src/model.c:2886-2907, 3612-3653): a layer whose records all name the
  other layer's codebooks gives the oracle's outputs for those records,
  decode and chunk; a selection whose records name different codebooks is
  refused with E_BOOKS (the caller's CPU path runs it), and one that does
  not touch such a record is unaffected.
- More than WARP_CRC_ERR_KEYS refused fills in one report window leave no
  key resident, and a lookahead fill refused by its checksum is reported by
  the next layer's chunk (E_CRC), never returned as a 0 with wrong outputs.
"""
import os
import struct

import numpy as np
import pytest

import container as ct
from gpu_util import BALANCED, dev, empty, host, log, open_ctx, rel_err
from oracle import pyoracle as po
from specs import SPECS

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture():
    return dict(np.load(os.path.join(HERE, "recchk.npz")))


def damaged(model, header, flip):
    rec = bytearray(model.layers[0].records[2])
    rec[:ct.HDR] = bytes(header)
    if flip == 1:
        rec[ct.HDR + 17] ^= 0x40
    elif flip == 2:
        rec[-1] ^= 0x40
    return np.frombuffer(bytes(rec), np.uint8)


def weights_only(ctx, model):
    """Codebooks and routers of every layer, no records."""
    S = ct.FMT_STAGES[model.spec.fmt]
    for L in range(model.spec.layers):
        lay = model.layers[L]
        ctx.set_codebooks(L, L * 3 * S, np.ascontiguousarray(model.books_raw[L * 3 * S:(L + 1) * 3 * S]))
        ctx.set_router(L, np.ascontiguousarray(lay.router, np.float32), lay.bias)


def expected_code(status, stricter):
    import warp_amd
    if stricter:
        return warp_amd.E_HEADER
    return {0: 0, 2: warp_amd.E_HEADER, 3: warp_amd.E_CRC}[int(status)]


@pytest.mark.parametrize("verify", [0, 1])
def test_refusals_match_the_reference(verify):
    import warp_amd
    g = fixture()
    names = [str(n) for n in g["names"]]
    ref = g["ref_verify1" if verify else "ref_verify0"]
    checked = 0
    for si, sname in enumerate(str(n) for n in g["spec_names"]):
        model = ct.build(SPECS[sname])
        for i in (i for i in range(len(names)) if int(g["spec"][i]) == si):
            rec = damaged(model, g["headers"][i], int(g["flips"][i]))
            L, e = int(g["layers"][i]), int(g["experts"][i])
            want = expected_code(ref[i], int(g["stricter"][i]))
            for path in ("put", "fetch"):
                # a context per case: an accepted record must not stay for the next one
                ctx = open_ctx(model, max_tokens=2, cache_slots=2, verify=bool(verify))
                try:
                    weights_only(ctx, model)
                    got = 0
                    try:
                        if path == "put":
                            ctx.put_expert(L, e, rec)
                        else:
                            ctx.set_fetch(lambda LL, ee: bytes(rec))
                            ctx.prefetch(L, [e])
                            ctx.sync()           # a refused checksum is reported by the next call that waits
                    except warp_amd.WarpHipError as ex:
                        got = ex.code
                    assert got == want, (names[i], path, verify, got, want)
                    assert bool(ctx.resident(L, e)) == (want == 0), (names[i], path)
                    checked += 1
                finally:
                    ctx.close()
    log(f"record_check (verify {verify}): {checked} put/fetch decisions equal the reference's "
        f"(3 stricter offset cases per spec refused by design)")


def with_codebook_id(rec, cbid):
    b = bytearray(rec)
    struct.pack_into("<H", b, 10, cbid)
    return bytes(b)


FOREIGN_SPEC = dict(hidden=256, inter=128, experts=16, top_k=4, layers=2, fmt="VQ3R", seed=313, **BALANCED)


def foreign_model(which):
    """Layer 0's records `which` (all when None) name layer 1's codebooks."""
    model = ct.build(ct.Spec(**FOREIGN_SPEC))
    S = ct.FMT_STAGES["VQ3R"]
    lay = model.layers[0]
    lay.records = [with_codebook_id(r, 3 * S) if (which is None or e in which) else r
                   for e, r in enumerate(lay.records)]
    return model


def test_records_decode_with_their_own_codebooks():
    import warp_amd
    model = foreign_model(None)
    ctx = open_ctx(model, max_tokens=8)
    try:
        warp_amd.load_container_model(ctx, model)
        lv = po.LayerView(model, 0)          # the oracle reads each record's codebook_id
        rng = np.random.default_rng(5)
        X = rng.normal(size=(8, FOREIGN_SPEC["hidden"])).astype(np.float32)
        for t in range(3):
            ref, ridx, _, _ = lv.moe_layer(X[t])
            out = empty(FOREIGN_SPEC["hidden"])
            idx, _ = ctx.moe_decode(0, dev(X[t]), out, want_route=True)
            assert np.array_equal(idx, ridx)
            assert rel_err(host(out), ref) <= 1e-4, rel_err(host(out), ref)
        # and not the layer's own codebooks: the same records with their ids
        # restored give other outputs
        plain = ct.build(ct.Spec(**FOREIGN_SPEC))
        assert rel_err(po.LayerView(plain, 0).moe_layer(X[0])[0], lv.moe_layer(X[0])[0]) > 1e-2
        ref, rroute, _ = lv.moe_chunk(X)
        out = empty((8, FOREIGN_SPEC["hidden"]))
        route, _ = ctx.moe_chunk(0, dev(X), out, 8, want_route=True)
        assert np.array_equal(route, rroute)
        assert rel_err(host(out), ref) <= 1e-4
        log("records naming layer 1's codebooks: decode and chunk equal the oracle (record codebook_id)")
    finally:
        ctx.close()


def test_mixed_codebooks_are_refused():
    import warp_amd
    plain = ct.build(ct.Spec(**FOREIGN_SPEC))
    lv = po.LayerView(plain, 0)
    rng = np.random.default_rng(6)
    X = rng.normal(size=(64, FOREIGN_SPEC["hidden"])).astype(np.float32)
    picks = [set(lv.moe_layer(x)[1].tolist()) for x in X]
    # one expert's record names other codebooks: the most often picked one
    counts = np.bincount([e for p in picks for e in p], minlength=16)
    odd = int(np.argmax(counts))
    with_odd = [t for t in range(64) if odd in picks[t]]
    without = [t for t in range(64) if odd not in picks[t]]
    assert with_odd and without
    model = foreign_model({odd})
    ctx = open_ctx(model, max_tokens=8)
    try:
        warp_amd.load_container_model(ctx, model)
        lvm = po.LayerView(model, 0)
        t = without[0]
        ref = lvm.moe_layer(X[t])[0]
        out = empty(FOREIGN_SPEC["hidden"])
        ctx.moe_decode(0, dev(X[t]), out, want_route=True)
        assert rel_err(host(out), ref) <= 1e-4
        for path in ("decode", "chunk"):
            with pytest.raises(warp_amd.WarpHipError) as ei:
                if path == "decode":
                    ctx.moe_decode(0, dev(X[with_odd[0]]), out, want_route=True)
                else:
                    Xc = np.ascontiguousarray(X[[without[0], with_odd[0]]])
                    ctx.moe_chunk(0, dev(Xc), empty((2, FOREIGN_SPEC["hidden"])), 2, want_route=True)
            assert ei.value.code == warp_amd.E_BOOKS, ei.value
        # a chunk of tokens that do not pick it computes
        Xc = np.ascontiguousarray(X[without[:4]])
        ref, _, _ = lvm.moe_chunk(Xc)
        out = empty((4, FOREIGN_SPEC["hidden"]))
        ctx.moe_chunk(0, dev(Xc), out, 4, want_route=True)
        assert rel_err(host(out), ref) <= 1e-4
        log(f"expert {odd} naming other codebooks: selections with it refused (E_BOOKS), others computed")
    finally:
        ctx.close()


def bad_crc(rec):
    b = bytearray(rec)
    struct.pack_into("<I", b, 36, struct.unpack_from("<I", b, 36)[0] ^ 1)
    return bytes(b)


def test_more_refusals_than_the_device_list_holds():
    import warp_amd
    spec = ct.Spec(hidden=64, inter=32, experts=256, top_k=2, layers=2, fmt="VQ3R", seed=17, shared_bits=0,
                   subnormals=False, keep_codes=False)
    model = ct.build(spec)
    recs = {(L, e): bad_crc(model.layers[L].records[e]) for L in range(2) for e in range(256)}
    ctx = open_ctx(model, max_tokens=2, cache_slots=512, verify=True)
    try:
        weights_only(ctx, model)
        ctx.set_fetch(lambda L, e: recs[(L, e)])
        ctx.prefetch(0, list(range(256)))
        ctx.prefetch(1, list(range(256)))
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.sync()
        assert ei.value.code == warp_amd.E_CRC
        st = ctx.cache_stats()
        assert st["resident"] == 0, st
        assert not any(ctx.resident(L, e) for L in range(2) for e in range(256))
        ctx.sync()                                       # reported once
        log("512 refused fills in one report: none left resident")
    finally:
        ctx.close()


def test_refused_lookahead_fill_fails_the_next_chunk():
    import warp_amd
    spec = ct.Spec(hidden=128, inter=64, experts=16, top_k=2, layers=2, fmt="VQ3R", seed=19, shared_bits=0)
    model = ct.build(spec)
    recs = {(L, e): model.layers[L].records[e] for L in range(2) for e in range(16)}
    for e in range(16):
        recs[(1, e)] = bad_crc(recs[(1, e)])
    ctx = open_ctx(model, max_tokens=4, cache_slots=32, verify=True, lookahead=16)
    try:
        weights_only(ctx, model)
        for e in range(16):
            ctx.put_expert(0, e, np.frombuffer(recs[(0, e)], np.uint8))
        ctx.set_fetch(lambda L, e: recs[(L, e)])
        X = np.random.default_rng(8).normal(size=(4, 128)).astype(np.float32)
        out = empty((4, 128))
        ctx.moe_chunk(0, dev(X), out, 4)                 # its lookahead claims all of layer 1
        with pytest.raises(warp_amd.WarpHipError) as ei:
            ctx.moe_chunk(1, dev(X), out, 4)
        assert ei.value.code in (warp_amd.E_CRC, warp_amd.E_MISSING), ei.value
        assert ctx.cache_stats()["resident"] == 16
        log("a lookahead fill refused by its checksum fails the next chunk (E_CRC)")
    finally:
        ctx.close()
