"""Synthetic expert containers in the reference's on-disk format.

Writes the files the reference loader reads (manifest.json, trunk.bin,
codebooks.bin, experts-L{L}.bin) and returns the same model in memory, so a
test can drive the compiled reference, the oracle and the HIP path from one
set of bytes. Deterministic for a given spec (numpy PCG64).

Layouts follow the reference's format documents and loader:
  - expert record: 48-byte header (src/waste_format.h:98-132), then the
    gate, up and down index blocks, then one fp16 scale per output row of
    each matrix, padded to 4 KiB (src/model.c:1698-1745);
  - index block: [row_block=64][position][row_in_block][slot]
    (docs/FORMAT.md:194-201); VQ4P packs four 6-bit codes in 3 bytes
    (docs/FORMAT.md:215-226); the VQ12 extension packs two 12-bit codes in
    the little-endian 24-bit word s0 | s1 << 12;
  - codebooks.bin: per (layer, kind, stage) a 16-byte header then
    entries x 8 fp16 (src/waste_format.h:139-150), ids base + kind*S + s;
  - trunk: F32 verbatim, Q8G/Q4G rows padded to whole groups then one fp16
    scale per group (src/model.c:529-669).
Only the shapes the loader validates for an all-MLA, all-MoE model are
written (src/model.c:711-790); attention weights are noise.
"""
from __future__ import annotations

import json
import os
import struct
import zlib
from dataclasses import dataclass, field

import numpy as np

FMT_CODE = {"VQ3R": 4, "VQ2R": 5, "VQ4P": 8, "VQ12": 9}
FMT_STAGES = {"VQ3R": 3, "VQ2R": 2, "VQ4P": 4, "VQ12": 2}
FMT_ENTRIES = {"VQ3R": 256, "VQ2R": 256, "VQ4P": 64, "VQ12": 4096}
FMT_SLOT = {"VQ3R": 3, "VQ2R": 2, "VQ4P": 3, "VQ12": 3}
FMT_INDEX_BITS = {"VQ3R": 8, "VQ2R": 8, "VQ4P": 6, "VQ12": 12}
TILE = 64
ALIGN = 4096
MAGIC_EXPERT = 0x50584557
MAGIC_CODEBOOK = 0x4B424357
HDR = 48


@dataclass
class Spec:
    hidden: int = 128
    inter: int = 64
    experts: int = 8
    top_k: int = 2
    layers: int = 2
    fmt: str = "VQ3R"
    router: str = "f32"          # "f32" | "q8" | "q4"
    router_std: float = 0.02
    bias: bool = True
    renorm: bool = True
    routed_scale: float = 2.0
    shared_bits: int = 8         # 8, 4, or 0 for no shared expert
    shared_group: int = 32
    shared_scale: tuple = (0.002, 0.02)   # per-group fp16 scale range of the shared expert
    n_shared: int = 1
    act: str = "silu"            # "silu" | "situ"
    situ_beta: float = 4.0
    situ_lbeta: float = 2.0
    book_std: float = 0.02
    subnormals: bool = True      # plant fp16 subnormals in codebooks and scales
    vocab: int = 64
    seed: int = 0
    keep_codes: bool = True      # keep the per-matrix code arrays (small shapes)
    dup_rows: tuple = ()         # (a, b): router row b is a copy of row a (exact ties)
    materialize: tuple = ()      # expert ids that get records; () = all (large shapes)
    latent: int = 0              # routed_expert_hidden_size: experts on a latent projection (0 = none)
    latent_norm: bool = True     # latent_moe_use_norm (with latent)


def index_bytes(fmt: str, M: int, N: int) -> int:
    return ((M + TILE - 1) // TILE) * (N // 8) * TILE * FMT_SLOT[fmt]


def pack_indices(fmt: str, codes: np.ndarray, M: int, N: int) -> bytes:
    """codes: [S][M][nv] ints -> blocked index block."""
    S, nv = FMT_STAGES[fmt], N // 8
    nb = (M + TILE - 1) // TILE
    full = np.zeros((S, nb * TILE, nv), dtype=np.uint32 if fmt in ("VQ4P", "VQ12") else np.uint8)
    full[:, :M, :] = codes
    # [S][nb][64][nv] -> [nb][nv][64][S]
    c = full.reshape(S, nb, TILE, nv).transpose(1, 3, 2, 0)
    if fmt in ("VQ3R", "VQ2R"):
        return c.astype(np.uint8).tobytes()
    if fmt == "VQ4P":
        s0, s1, s2, s3 = (c[..., k] & 0x3F for k in range(4))
        b0 = (s0 | (s1 << 6)) & 0xFF
        b1 = ((s1 >> 2) | (s2 << 4)) & 0xFF
        b2 = ((s2 >> 4) | (s3 << 2)) & 0xFF
    else:  # VQ12
        w = (c[..., 0].astype(np.uint32) & 0xFFF) | ((c[..., 1].astype(np.uint32) & 0xFFF) << 12)
        b0, b1, b2 = w & 0xFF, (w >> 8) & 0xFF, (w >> 16) & 0xFF
    return np.stack([b0, b1, b2], axis=-1).astype(np.uint8).tobytes()


def f16_bits(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def quant_rows(rng, rows: int, N: int, bits: int, group: int, scale=(0.002, 0.02)):
    """Q8G/Q4G payload (rows padded to whole groups) and per-group fp16 scales."""
    ng = (N + group - 1) // group
    n = ng * group
    if bits == 8:
        q = rng.integers(-127, 128, size=(rows, n), dtype=np.int64)
        payload = (q & 0xFF).astype(np.uint8)
        rowbytes = n
    else:
        v = rng.integers(-8, 8, size=(rows, n), dtype=np.int64)
        lo, hi = v[:, 0::2] + 8, v[:, 1::2] + 8
        payload = (lo | (hi << 4)).astype(np.uint8)
        rowbytes = n // 2
    scales = f16_bits(rng.uniform(scale[0], scale[1], size=(rows, ng)))
    return payload.reshape(rows, rowbytes), scales.reshape(rows, ng), rowbytes


@dataclass
class Layer:
    router: np.ndarray                   # [E][H] f32 (dequantised view if quantised)
    router_q: tuple | None               # (payload, scales, rowbytes, bits, group)
    bias: np.ndarray | None              # [E] f32
    shared: list = field(default_factory=list)  # [(payload, scales, rowbytes)] gate, up, down
    codes: list = field(default_factory=list)   # per expert: [gate, up, down] code arrays [S][M][nv]
    scales: list = field(default_factory=list)  # per expert: [gate, up, down] fp16 bits
    records: list = field(default_factory=list)  # per expert: bytes (whole record)
    # latent MoE: (down (payload, scales, rowbytes, bits, group) [lat][H],
    # up [H][lat], norm weight [lat] f32 or None), or None
    latent: tuple | None = None


@dataclass
class Model:
    spec: Spec
    books_raw: np.ndarray                # [n_books][E][8] uint16
    layers: list
    rec_bytes: int

    def cb_base(self, L: int) -> int:
        return L * 3 * FMT_STAGES[self.spec.fmt]


def build(spec: Spec) -> Model:
    rng = np.random.Generator(np.random.PCG64(spec.seed))
    S, E = FMT_STAGES[spec.fmt], FMT_ENTRIES[spec.fmt]
    H, I = spec.hidden, spec.inter
    Hx = spec.latent or H                # the experts' width
    n_books = spec.layers * 3 * S
    books = rng.normal(0.0, spec.book_std, size=(n_books, E, 8)).astype(np.float16)
    if spec.subnormals:
        # fp16 subnormals: flushed to +-0 at codebook load, kept in scales
        books[0, 1, :3] = np.float16(3.0e-6)
        books[0, 2, 5] = np.float16(-4.0e-5)
        books[-1, E - 1, 7] = np.float16(1.0e-7)
    books_raw = books.view(np.uint16)
    shapes = [(I, Hx), (I, Hx), (Hx, I)]
    layers = []
    rec_len = HDR + sum(index_bytes(spec.fmt, M, N) for M, N in shapes) + 2 * (2 * I + Hx)
    rec_bytes = (rec_len + ALIGN - 1) // ALIGN * ALIGN
    for L in range(spec.layers):
        router = rng.normal(0.0, spec.router_std, size=(spec.experts, H)).astype(np.float32)
        router_q = None
        if spec.router != "f32":
            bits = 8 if spec.router == "q8" else 4
            router_q = quant_rows(rng, spec.experts, H, bits, 128) + (bits, 128)
        if spec.dup_rows:
            a, b = spec.dup_rows
            router[b] = router[a]
        bias = rng.normal(0.0, 0.01, size=spec.experts).astype(np.float32) if spec.bias else None
        shared = []
        if spec.shared_bits:
            si = I * spec.n_shared
            for (M, N) in [(si, H), (si, H), (H, si)]:
                shared.append(quant_rows(rng, M, N, spec.shared_bits, spec.shared_group, spec.shared_scale))
        latent = None
        if spec.latent:
            dq = quant_rows(rng, Hx, H, 8, 128) + (8, 128)
            uq = quant_rows(rng, H, Hx, 8, 128) + (8, 128)
            nw = rng.uniform(0.5, 1.5, size=Hx).astype(np.float32) if spec.latent_norm else None
            latent = (dq, uq, nw)
        lay = Layer(router=router, router_q=router_q, bias=bias, shared=shared, latent=latent)
        for e in range(spec.experts):
            if spec.materialize and e not in spec.materialize:
                lay.codes.append(None)
                lay.scales.append(None)
                lay.records.append(None)
                continue
            body = bytearray()
            offs = []
            codes_e, scales_e = [], []
            for (M, N) in shapes:
                c = rng.integers(0, E, size=(S, M, N // 8), dtype=np.uint16)
                if spec.keep_codes:
                    codes_e.append(c)
                offs.append(HDR + len(body))
                body += pack_indices(spec.fmt, c, M, N)
            corr = HDR + len(body)
            for k, (M, _N) in enumerate(shapes):
                s = f16_bits(rng.uniform(0.01, 0.05, size=M))
                if spec.subnormals and e == 0 and k == 0:
                    s[min(3, M - 1)] = f16_bits(np.float16(2.0e-5))  # subnormal scale
                scales_e.append(s)
                body += s.tobytes()
            hdr = struct.pack("<IHHBBHHHIIIIIIII", MAGIC_EXPERT, L, e, FMT_CODE[spec.fmt], 0,
                              L * 3 * S, 0, 0, rec_bytes // ALIGN, offs[0], offs[1], offs[2],
                              corr, zlib.crc32(bytes(body)) & 0xFFFFFFFF, 0, 0)
            rec = hdr + bytes(body)
            rec += b"\0" * (rec_bytes - len(rec))
            lay.codes.append(codes_e)
            lay.scales.append(scales_e)
            lay.records.append(rec)
        layers.append(lay)
    return Model(spec=spec, books_raw=books_raw, layers=layers, rec_bytes=rec_bytes)


class _Trunk:
    def __init__(self, rng):
        self.buf = bytearray()
        self.index = []
        self.rng = rng

    def f32(self, name, arr):
        off = len(self.buf)
        self.buf += np.asarray(arr, dtype=np.float32).tobytes()
        self.index.append({"name": name, "fmt": 0, "off": off, "shape": list(np.shape(arr)),
                           "bytes": len(self.buf) - off})

    def quant(self, name, shape, q=None):
        rows = int(np.prod(shape[:-1]))
        if q is None:
            q = quant_rows(self.rng, rows, shape[-1], 8, 128) + (8, 128)
        payload, scales, _rowbytes, bits, group = q
        off = len(self.buf)
        self.buf += payload.tobytes()
        soff = len(self.buf)
        self.buf += scales.tobytes()
        self.index.append({"name": name, "fmt": 2 if bits == 8 else 3, "off": off,
                           "shape": list(shape), "group": group, "scale_off": soff,
                           "bytes": len(self.buf) - off})


def digest(model: Model) -> str:
    """sha256 over every byte the model defines (codebooks, routers, biases,
    shared experts, records), to catch a generator that drifted."""
    import hashlib
    h = hashlib.sha256()
    h.update(model.books_raw.tobytes())
    for lay in model.layers:
        h.update(np.ascontiguousarray(lay.router).tobytes())
        if lay.router_q is not None:
            h.update(lay.router_q[0].tobytes())
            h.update(lay.router_q[1].tobytes())
        if lay.bias is not None:
            h.update(lay.bias.tobytes())
        for q in lay.shared:
            h.update(q[0].tobytes())
            h.update(q[1].tobytes())
        if lay.latent is not None:
            for q in lay.latent[:2]:
                h.update(q[0].tobytes())
                h.update(q[1].tobytes())
            if lay.latent[2] is not None:
                h.update(lay.latent[2].tobytes())
        for r in lay.records:
            if r is not None:
                h.update(r)
    return h.hexdigest()


def write(model: Model, out: str) -> str:
    """Write `model` as a container directory the reference loader accepts
    (formats the reference refuses, such as VQ12, are still written the same
    way for this build's own readers)."""
    spec = model.spec
    os.makedirs(out, exist_ok=True)
    rng = np.random.Generator(np.random.PCG64(spec.seed + 1000))
    S, E = FMT_STAGES[spec.fmt], FMT_ENTRIES[spec.fmt]
    H, I = spec.hidden, spec.inter
    nh, nope, rope, vh, kvl = 2, 16, 8, 16, 32
    cfg = {
        "model_type": "kimi_linear", "architectures": ["KimiLinearForCausalLM"],
        "hidden_size": H, "num_hidden_layers": spec.layers, "first_k_dense_replace": 0,
        "intermediate_size": 2 * I, "moe_intermediate_size": I,
        "num_experts": spec.experts, "num_experts_per_token": spec.top_k,
        "num_shared_experts": spec.n_shared, "routed_scaling_factor": spec.routed_scale,
        "num_attention_heads": nh, "qk_nope_head_dim": nope, "qk_rope_head_dim": rope,
        "v_head_dim": vh, "kv_lora_rank": kvl, "q_lora_rank": None, "mla_use_nope": True,
        "rms_norm_eps": 1e-5, "vocab_size": spec.vocab, "tie_word_embeddings": False,
        "bos_token_id": 1, "eos_token_id": 2,
    }
    if spec.renorm:
        cfg["moe_renormalize"] = True
    if spec.latent:
        cfg["routed_expert_hidden_size"] = spec.latent
        if spec.latent_norm:
            cfg["latent_moe_use_norm"] = True
    if spec.act == "situ":
        cfg["hidden_act"] = "situ"
        cfg["activation_situ_beta"] = spec.situ_beta
        cfg["activation_situ_linear_beta"] = spec.situ_lbeta
    t = _Trunk(rng)
    t.quant("model.embed_tokens.weight", [spec.vocab, H])
    for L, lay in enumerate(model.layers):
        p = f"model.layers.{L}."
        t.f32(p + "input_layernorm.weight", np.ones(H, np.float32))
        t.f32(p + "post_attention_layernorm.weight", np.ones(H, np.float32))
        a = p + "self_attn."
        t.quant(a + "q_proj.weight", [nh * (nope + rope), H])
        t.quant(a + "kv_a_proj_with_mqa.weight", [kvl + rope, H])
        t.f32(a + "kv_a_layernorm.weight", np.ones(kvl, np.float32))
        t.quant(a + "kv_b_proj.weight", [nh * (nope + vh), kvl])
        t.quant(a + "o_proj.weight", [H, nh * vh])
        m = p + "block_sparse_moe."
        if lay.router_q is None:
            t.f32(m + "gate.weight", lay.router)
        else:
            t.quant(m + "gate.weight", [spec.experts, H], lay.router_q)
        if lay.bias is not None:
            t.f32(m + "gate.e_score_correction_bias", lay.bias)
        if lay.shared:
            si = I * spec.n_shared
            for nm, shp, q in zip(("gate_proj", "up_proj", "down_proj"),
                                  ([si, H], [si, H], [H, si]), lay.shared):
                t.quant(m + f"shared_experts.{nm}.weight", shp,
                        q + (spec.shared_bits, spec.shared_group))
        if lay.latent is not None:
            dq, uq, nw = lay.latent
            t.quant(m + "routed_expert_down_proj.weight", [spec.latent, H], dq)
            t.quant(m + "routed_expert_up_proj.weight", [H, spec.latent], uq)
            if nw is not None:
                t.f32(m + "routed_expert_norm.weight", nw)
    t.f32("model.norm.weight", np.ones(H, np.float32))
    t.quant("lm_head.weight", [spec.vocab, H])
    with open(os.path.join(out, "trunk.bin"), "wb") as f:
        f.write(t.buf)
    with open(os.path.join(out, "codebooks.bin"), "wb") as f:
        for b in range(model.books_raw.shape[0]):
            f.write(struct.pack("<IHBBII", MAGIC_CODEBOOK, b & 0xFFFF, FMT_CODE[spec.fmt], 8, E, 0))
            f.write(model.books_raw[b].tobytes())
    layers = {}
    for L, lay in enumerate(model.layers):
        name = f"experts-L{L}.bin"
        with open(os.path.join(out, name), "wb") as f:
            for rec in lay.records:
                f.write(rec)
        layers[str(L)] = {"file": name, "experts": spec.experts,
                          "bytes": spec.experts * model.rec_bytes, "codebook_base": L * 3 * S}
    manifest = {
        "format_version": 0, "arch": cfg["model_type"], "tensor_prefix": "", "config": cfg,
        "expert_quant": {"fmt": spec.fmt, "stages": S, "vec_dim": 8, "entries": E,
                         "index_block": TILE, "bits_per_weight": 3,
                         "index_bits": FMT_INDEX_BITS[spec.fmt]},
        "layers": layers, "trunk": t.index,
    }
    with open(os.path.join(out, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    return out
