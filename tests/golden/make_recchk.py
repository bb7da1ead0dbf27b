#!/usr/bin/env python3
"""Writes tests/golden/recchk.npz: the compiled reference's record_check
(src/model.c:1698-1745, through oracle/_ref) on one record with its header
or payload damaged one way per case, once with the checksum off and once
with it on. Run in a container that has the reference sources; the fixture
is data and travels without them.

Each case is a (spec, layer, expert) record of the synthetic containers of
specs.py, the 48-byte header to put in front of its payload, whether a
payload byte is flipped, and the (layer, expert) the check is asked for.
The fixture keeps the headers and the reference's verdicts (0 OK,
2 E_HEADER, 3 E_CRC); the records themselves are rebuilt from the specs.
"""
import os
import struct
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

# header fields: name -> (byte offset, struct code) of waste_expert_hdr
# (src/waste_format.h:98-132)
FIELDS = {"magic": (0, "<I"), "layer": (4, "<H"), "expert": (6, "<H"), "fmt": (8, "<B"),
          "codebook_id": (10, "<H"), "lowrank_id": (12, "<H"), "blocks": (16, "<I"), "gate_off": (20, "<I"),
          "up_off": (24, "<I"), "down_off": (28, "<I"), "corr_off": (32, "<I"), "crc": (36, "<I")}


def field(h: bytes, name: str) -> int:
    o, f = FIELDS[name]
    return struct.unpack_from(f, h, o)[0]


def with_fields(h: bytes, **kv) -> bytes:
    b = bytearray(h)
    for k, v in kv.items():
        o, f = FIELDS[k]
        struct.pack_into(f, b, o, v)
    return bytes(b)


def cases_for(name: str, model):
    """(case name, header, flip payload byte, asked layer, asked expert,
    stricter here): the record is expert 2 of layer 0."""
    spec = model.spec
    rec = model.layers[0].records[2]
    h = rec[:ct.HDR]
    S = ct.FMT_STAGES[spec.fmt]
    n_books = spec.layers * 3 * S
    rb = model.rec_bytes
    Hx = spec.latent or spec.hidden
    scales = 2 * (2 * spec.inter + Hx)
    g, u, d, cc = (field(h, k) for k in ("gate_off", "up_off", "down_off", "corr_off"))
    out = [
        ("ok", h, 0, 0, 2, 0),
        ("magic", with_fields(h, magic=field(h, "magic") ^ 1), 0, 0, 2, 0),
        ("layer_field", with_fields(h, layer=1), 0, 0, 2, 0),
        ("expert_field", with_fields(h, expert=3), 0, 0, 2, 0),
        ("asked_other_expert", h, 0, 0, 5, 0),
        ("asked_other_layer", h, 0, 1, 2, 0),
        ("blocks_plus", with_fields(h, blocks=field(h, "blocks") + 1), 0, 0, 2, 0),
        ("blocks_zero", with_fields(h, blocks=0), 0, 0, 2, 0),
        ("fmt_vq3r", with_fields(h, fmt=4), 0, 0, 2, 0),
        ("fmt_vq2r", with_fields(h, fmt=5), 0, 0, 2, 0),
        ("fmt_vq4p", with_fields(h, fmt=8), 0, 0, 2, 0),
        ("fmt_unknown", with_fields(h, fmt=7), 0, 0, 2, 0),
        ("lowrank", with_fields(h, lowrank_id=1), 0, 0, 2, 0),
        ("codebook_last_set", with_fields(h, codebook_id=n_books - 3 * S), 0, 0, 2, 0),
        ("codebook_past_end", with_fields(h, codebook_id=n_books - 3 * S + 1), 0, 0, 2, 0),
        ("codebook_huge", with_fields(h, codebook_id=0xFFFF), 0, 0, 2, 0),
        ("gate_off_moved", with_fields(h, gate_off=g + 4), 0, 0, 2, 0),
        ("up_eq_gate", with_fields(h, up_off=g), 0, 0, 2, 0),
        ("down_eq_up", with_fields(h, down_off=u), 0, 0, 2, 0),
        ("corr_eq_down", with_fields(h, corr_off=d), 0, 0, 2, 0),
        ("corr_past_end", with_fields(h, corr_off=rb + 1), 0, 0, 2, 0),
        ("scales_past_end", with_fields(h, corr_off=rb - scales + 2), 0, 0, 2, 0),
        ("scales_at_end", with_fields(h, corr_off=rb - scales), 0, 0, 2, 0),
        ("crc_field", with_fields(h, crc=field(h, "crc") ^ 0x10), 0, 0, 2, 0),
        ("payload_flip", h, 1, 0, 2, 0),
        ("padding_flip", h, 2, 0, 2, 0),
        # increasing offsets with blocks shorter than the shape: the
        # reference reads the next block's bytes; the kernels here index a
        # block's whole shape, so this build refuses them (E_HEADER)
        ("up_overlaps_gate", with_fields(h, up_off=g + 8), 0, 0, 2, 1),
        ("down_overlaps_up", with_fields(h, down_off=u + 8), 0, 0, 2, 1),
        ("corr_overlaps_down", with_fields(h, corr_off=d + 8), 0, 0, 2, 1),
    ]
    return [(f"{name}:{c[0]}",) + c[1:] for c in out]


def damaged(model, header: bytes, flip: int) -> bytes:
    rec = bytearray(model.layers[0].records[2])
    rec[:ct.HDR] = header
    if flip == 1:       # a byte of the payload (checksummed)
        rec[ct.HDR + 17] ^= 0x40
    elif flip == 2:     # a byte past the scales (not checksummed)
        rec[-1] ^= 0x40
    return bytes(rec)


SPEC_NAMES = ("vq3r_f32", "vq4p_f32")


def main():
    names, headers, flips, layers, experts, stricter, st0, st1, spec_ix = [], [], [], [], [], [], [], [], []
    for si, sname in enumerate(SPEC_NAMES):
        model = ct.build(SPECS[sname])
        d = tempfile.mkdtemp(prefix=f"recchk_{sname}_")
        ct.write(model, d)
        ref = po.Ref(d)
        for (cname, hdr, flip, L, e, strict) in cases_for(sname, model):
            rec = np.frombuffer(damaged(model, hdr, flip), np.uint8)
            names.append(cname)
            headers.append(np.frombuffer(hdr, np.uint8))
            flips.append(flip)
            layers.append(L)
            experts.append(e)
            stricter.append(strict)
            st0.append(ref.record_check(L, e, rec, 0))
            st1.append(ref.record_check(L, e, rec, 1))
            spec_ix.append(si)
        ref.close()
    path = os.path.join(HERE, "recchk.npz")
    np.savez_compressed(path, names=np.array(names), headers=np.stack(headers), flips=np.array(flips, np.int32),
                        layers=np.array(layers, np.int32), experts=np.array(experts, np.int32),
                        stricter=np.array(stricter, np.int32), ref_verify0=np.array(st0, np.int32),
                        ref_verify1=np.array(st1, np.int32), spec=np.array(spec_ix, np.int32),
                        spec_names=np.array(SPEC_NAMES))
    for n, a, b in zip(names, st0, st1):
        print(f"{n:40s} {a} {b}")


if __name__ == "__main__":
    main()
