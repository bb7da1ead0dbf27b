"""The oracle's record_check (or_record_check, oracle/oracle.c) against the
compiled reference's verdicts on tests/golden/recchk.npz: one damaged
header or payload per condition of src/model.c:1703-1738 (magic, identity,
block count, format label, lowrank_id, codebook_id bound, each offset order,
room for the scales, the payload checksum with verify off and on), on a
byte-code (VQ3R) and a VQ4P container. Where the reference sources are
built (oracle/_ref), its live verdicts are compared too."""
import os

import numpy as np
import pytest

import container as ct
from oracle import pyoracle as po
from specs import SPECS

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def damaged(model, header, flip):
    rec = bytearray(model.layers[0].records[2])
    rec[:ct.HDR] = bytes(header)
    if flip == 1:
        rec[ct.HDR + 17] ^= 0x40
    elif flip == 2:
        rec[-1] ^= 0x40
    return np.frombuffer(bytes(rec), np.uint8)


def test_fixture_covers_every_condition():
    g = dict(np.load(os.path.join(HERE, "recchk.npz")))
    # every outcome appears: accepted, refused by header, refused by checksum
    assert set(g["ref_verify0"].tolist()) == {0, 2}
    assert set(g["ref_verify1"].tolist()) == {0, 2, 3}
    assert len(g["names"]) == 58


@pytest.mark.parametrize("verify", [0, 1])
def test_oracle_record_check_matches_the_reference(verify):
    g = dict(np.load(os.path.join(HERE, "recchk.npz")))
    ref = g["ref_verify1" if verify else "ref_verify0"]
    live = os.path.exists(po.REF_LIB)
    for si, sname in enumerate(str(n) for n in g["spec_names"]):
        spec = SPECS[sname]
        model = ct.build(spec)
        S = ct.FMT_STAGES[spec.fmt]
        m = [spec.inter, spec.inter, spec.latent or spec.hidden]
        r = None
        if live:
            import tempfile
            d = tempfile.mkdtemp(prefix=f"recchk_{sname}_")
            ct.write(model, d)
            r = po.Ref(d)
        try:
            for i in np.flatnonzero(g["spec"] == si):
                rec = damaged(model, g["headers"][i], int(g["flips"][i]))
                L, e = int(g["layers"][i]), int(g["experts"][i])
                got = po.record_check(rec, L, e, spec.fmt, S, spec.layers * 3 * S, m, verify)
                assert got == int(ref[i]), (str(g["names"][i]), verify, got, int(ref[i]))
                if r is not None:
                    assert r.record_check(L, e, rec, verify) == int(ref[i]), str(g["names"][i])
        finally:
            if r is not None:
                r.close()
