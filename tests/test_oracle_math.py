"""Pins for what the compiled reference cannot run or does not check: the
2 x 4096 12-bit format, the fp16 conversions' edge cases, the encoder, the
crc32 and the routing rules. Each check is an independent computation (a
closed form, a library routine, brute force), not the oracle's own formula."""
import zlib

import numpy as np
import pytest

import container as ct
from oracle import pyoracle as po


def test_crc32_known_answer():
    assert po.lib().or_crc32(b"123456789", 9) == 0xCBF43926
    data = np.random.default_rng(0).integers(0, 256, 5000, dtype=np.uint8).tobytes()
    assert po.lib().or_crc32(data, len(data)) == zlib.crc32(data)


def test_f16_conversions():
    L = po.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float64)
    keep = np.array([L.or_f16_keep(int(v)) for v in h[::7]])
    flush = np.array([L.or_f16_flush(int(v)) for v in h[::7]])
    ff = f[::7]
    exp = (h[::7] >> 10) & 0x1F
    normal = (exp > 0) & (exp < 31)
    sub = exp == 0
    # normal numbers are exact in both; subnormals kept exactly or flushed to 0
    assert np.array_equal(keep[normal], ff[normal])
    assert np.array_equal(flush[normal], ff[normal])
    assert np.array_equal(keep[sub], ff[sub])
    assert np.all(flush[sub] == 0.0)
    # exponent 31 is rebiased as a normal number, not inf/nan (src/simd.h:64)
    assert L.or_f16_keep(0x7C00) == 65536.0 and L.or_f16_flush(0x7C01) == 65536.0 * (1 + 2 ** -10)


def _vq12_case(seed, M=64, N=128):
    spec = ct.Spec(hidden=N, inter=M, experts=1, top_k=1, layers=1, fmt="VQ12", seed=seed,
                   shared_bits=0, subnormals=True)
    return spec, ct.build(spec)


def test_vq12_matvec_against_float64_decode():
    spec, model = _vq12_case(5)
    books = po.books_flat(model.books_raw)                      # flushed, [book][entry][8]
    rec = np.frombuffer(model.layers[0].records[0], np.uint8)
    hdr = np.frombuffer(model.layers[0].records[0][:48], np.uint32)
    codes = model.layers[0].codes[0]
    for kind in range(3):
        M, N = (spec.inter, spec.hidden) if kind < 2 else (spec.hidden, spec.inter)
        soff = [0, spec.inter, 2 * spec.inter][kind]
        scale = rec[int(hdr[8]) + 2 * soff:int(hdr[8]) + 2 * (soff + M)].view(np.uint16).copy()
        c = codes[kind]                                          # [2][M][nv]
        W = (books[kind * 2 + 0][c[0]].astype(np.float64) + books[kind * 2 + 1][c[1]]).reshape(M, N)
        s = scale.view(np.float16).astype(np.float64)
        x = np.random.default_rng(kind).normal(size=N).astype(np.float32)
        ref = (W * s[:, None]) @ x.astype(np.float64)
        y = po.vq_matvec("VQ12", rec[int(hdr[5 + kind]):].copy(), scale, x, po.books_T(model.books_raw),
                         kind * 2, M, N)
        assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))
        # the decoded weights are the closed form, bit for bit
        Wd = po.decode_weights("VQ12", rec[int(hdr[5 + kind]):].copy(), scale, books, kind * 2, M, N)
        W32 = (books[kind * 2 + 0][c[0]] + books[kind * 2 + 1][c[1]]).reshape(M, N).astype(np.float32)
        Wexp = (W32 * s.astype(np.float32)[:, None]).astype(np.float32)
        assert np.array_equal(Wd.view(np.uint32), Wexp.view(np.uint32))


def test_vq12_reduces_to_vq2r_for_byte_codes():
    """With every code < 256 and the first 256 entries of each 4096-entry book
    equal to a VQ2R book, the 12-bit path must give VQ2R's result bit for bit
    (VQ2R is a format the reference runs)."""
    rng = np.random.default_rng(9)
    M, N = 64, 128
    nv = N // 8
    b256 = rng.normal(0, 0.02, size=(2, 256, 8)).astype(np.float16).view(np.uint16)
    b4096 = rng.normal(0, 0.02, size=(2, 4096, 8)).astype(np.float16).view(np.uint16)
    b4096[:, :256] = b256
    codes = rng.integers(0, 256, size=(2, M, nv))
    idx2 = np.frombuffer(ct.pack_indices("VQ2R", codes, M, N), np.uint8).copy()
    idx12 = np.frombuffer(ct.pack_indices("VQ12", codes, M, N), np.uint8).copy()
    scale = rng.uniform(0.01, 0.05, M).astype(np.float16).view(np.uint16)
    x = rng.normal(size=N).astype(np.float32)
    y2 = po.vq_matvec("VQ2R", idx2, scale, x, po.books_T(b256), 0, M, N)
    y12 = po.vq_matvec("VQ12", idx12, scale, x, po.books_T(b4096), 0, M, N)
    assert np.array_equal(y2.view(np.uint32), y12.view(np.uint32))


@pytest.mark.parametrize("fmt", ["VQ3R", "VQ2R", "VQ4P", "VQ12"])
def test_code_packing_round_trip(fmt):
    rng = np.random.default_rng(1)
    M, N = 70, 64                                                 # a ragged row block
    S, E = ct.FMT_STAGES[fmt], ct.FMT_ENTRIES[fmt]
    codes = rng.integers(0, E, size=(S, M, N // 8))
    idx = np.frombuffer(ct.pack_indices(fmt, codes, M, N), np.uint8).copy()
    assert idx.nbytes == po.lib().or_index_bytes(po.FMT[fmt], M, N)
    for r in (0, 63, 64, 69):
        for v in (0, N // 8 - 1):
            for s in range(S):
                assert po.lib().or_code_at(po.FMT[fmt], idx.ctypes.data, N, r, v, s) == codes[s, r, v]


def test_encoder_first_minimum_and_residual():
    """waste_vq_encode semantics: per stage the nearest entry (strict <, so a
    duplicate later entry never wins), then the residual feeds the next stage."""
    rng = np.random.default_rng(4)
    E, S = 64, 2
    books = rng.normal(0, 1, size=(S, E, 8)).astype(np.float32)
    books[0, 40] = books[0, 7]                                    # duplicate: 7 must win
    a, b = 7, 19
    X = (books[0, a] + books[1, b] * np.float32(1e-3))[None, :].astype(np.float32)
    out = np.empty((1, S), np.uint16)
    po.lib().or_vq_encode(X.ctypes.data, 1, books.ctypes.data, S, E, 8, out.ctypes.data)
    assert out[0, 0] == a
    # brute force over stage 1 on the exact residual
    resid = X[0] - books[0, a]
    d = ((resid[None, :] - books[1]) ** 2).sum(1)
    assert out[0, 1] == int(np.argmin(d))


def test_route_rules():
    logits = np.array([0.5, 2.0, 2.0, -1.0, 2.0, 0.1], np.float32)
    idx, w, sc = po.route(logits, None, 3, 0, 1, 1.0)
    assert list(idx) == [1, 2, 4]                                 # equal scores: lowest id first
    s = 1 / (1 + np.exp(-np.float64(2.0)))
    assert np.allclose(w, [1 / 3] * 3, rtol=1e-6) and abs(sc[1] - s) < 1e-7
    bias = np.array([3.0, 0, 0, 0, 0, 0], np.float32)             # bias selects, weight stays unbiased
    idx, w, sc = po.route(logits, bias, 1, 0, 0, 2.0)
    assert idx[0] == 0 and np.isclose(w[0], 2.0 * sc[0])
    # softmax extension: same order for monotone scores, weights are probabilities
    idx, w, sc = po.route(logits, None, 2, 1, 0, 1.0)
    assert list(idx) == [1, 2] and abs(sc.sum() - 1.0) < 1e-6


@pytest.mark.parametrize("E,K,renorm,scale,spread", [(256, 8, 0, 1.0, 3.0), (256, 8, 1, 2.5, 1.0),
                                                     (384, 16, 1, 1.0, 0.05), (64, 4, 0, 0.7, 8.0)])
def test_softmax_route_against_float64(E, K, renorm, scale, spread):
    """The softmax routing extension against a float64 softmax computed here
    (exp of the max-subtracted logits over their sum): each score within the
    rounding of one exp, an E-term sequential fp32 sum and one division; the
    picks are the top K of score + bias (bias selects, the weights stay
    unbiased); the weights renormalised when asked and scaled. A base-2 exp,
    a temperature, exp of the biased logits, biased weights or a missing
    renormalisation each miss these bounds by orders of magnitude."""
    rng = np.random.default_rng(E + K + renorm)
    logits = (rng.standard_normal(E) * spread).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.02).astype(np.float32)
    idx, w, sc = po.route(logits, bias, K, 1, renorm, scale)
    l64 = logits.astype(np.float64)
    p = np.exp(l64 - l64.max())
    p /= p.sum()
    tol = (E + 4) * 2.0 ** -24
    assert np.all(np.abs(sc - p) <= tol * p + 2.0 ** -149), float(np.max(np.abs(sc - p) / p))
    order = sorted(range(E), key=lambda e: (-(p[e] + float(bias[e])), e))[:K]
    assert list(idx) == order
    wr = p[order]
    if renorm:
        wr = wr / wr.sum()
    wr = wr * scale
    assert np.allclose(w, wr, rtol=tol + 2.0 ** -22, atol=0), float(np.max(np.abs(w - wr) / wr))


def test_sigmoid_route_against_float64():
    """The reference's sigmoid scores (src/model.c:2723-2725) against float64:
    within 2 ulp of 1/(1+exp(-x)); picks the top K of score + bias."""
    rng = np.random.default_rng(5)
    E, K = 384, 16
    logits = (rng.standard_normal(E) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    idx, w, sc = po.route(logits, bias, K, 0, 1, 2.5)
    p = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    assert np.all(np.abs(sc - p) <= 4 * 2.0 ** -24 * p)
    order = sorted(range(E), key=lambda e: (-(p[e] + float(bias[e])), e))[:K]
    assert list(idx) == order
    wr = p[order] / p[order].sum() * 2.5
    assert np.allclose(w, wr, rtol=(K + 4) * 2.0 ** -24, atol=0)


def test_device_expf_is_glibc_on_every_float():
    """The kernels' expf (warp_amd/csrc/expf_glibc.h, compiled here as C)
    against the host's glibc expf on all 2^32 inputs, bit for bit. The
    reference scores its router logits and computes SiLU with glibc's expf
    (src/model.c:2724, :501), which is not correctly rounded; a correctly
    rounded exp, or the same algorithm without the fused range reduction,
    differs from it on some inputs."""
    import os
    first = np.zeros(1, np.uint32)
    n = po.lib().or_expf_mismatches(0, 1 << 32, max(1, min(os.cpu_count() or 1, 16)), first.ctypes.data)
    assert n == 0, f"{n} inputs differ, first 0x{int(first[0]):08x}"
    # the comparison is sensitive: a correctly rounded exp misses glibc on this sample
    x = np.random.default_rng(0).uniform(-100, 80, 1 << 20).astype(np.float32)
    gl = np.empty_like(x)
    po.lib().or_expf_array(x.ctypes.data, gl.ctypes.data, len(x))
    cr = np.exp(x.astype(np.float64)).astype(np.float32)
    assert np.count_nonzero(cr.view(np.uint32) != gl.view(np.uint32)) > 0


def test_glibc_expf_is_monotone():
    """glibc's expf never decreases from one float to the next, over every
    float from -inf to +inf (the device's warp_expf is the same function, by
    the test above). The certified router bounds a score by the scores at
    its logit interval's ends when the logits are large, which rests on this
    (the add and the division that follow are correctly rounded, so
    monotone). The walk visits the 2^32 - 2^24 + 2 non-NaN patterns in
    value order (-0 and +0 both)."""
    import os
    assert po.lib().or_expf_decreases(max(1, min(os.cpu_count() or 1, 16))) == 0


def test_kda_step_against_float64():
    """The KDA recurrence in float64 (q, k L2-normalised, q by 1/sqrt(K);
    S <- diag(exp g) S; d = beta (v - S^T k); S <- S + k d^T; o = S^T q)
    against the oracle's fp32 step: a transposed state, a missing decay,
    the update before the readout or an unnormalised key fail by far more
    than fp32 rounding."""
    rng = np.random.default_rng(21)
    H, K, V = 3, 32, 48
    q, k = rng.normal(size=(1, H, K)), rng.normal(size=(1, H, K))
    v, g = rng.normal(size=(1, H, V)), -rng.uniform(0, 2, size=(1, H, K))
    beta, S0 = rng.uniform(0, 1, size=(1, H)), rng.normal(size=(H, K, V)) * 0.1
    f32 = lambda a: np.asarray(a, np.float32)
    S, o = po.kda_forward(f32(q), f32(k), f32(v), f32(g), f32(beta), f32(S0))
    for h in range(H):
        qn = q[0, h] / np.sqrt((q[0, h] ** 2).sum() + 1e-12) / np.sqrt(K)
        kn = k[0, h] / np.sqrt((k[0, h] ** 2).sum() + 1e-12)
        Sh = np.exp(g[0, h])[:, None] * f32(S0[h]).astype(np.float64)
        d = beta[0, h] * (v[0, h] - Sh.T @ kn)
        Sh = Sh + np.outer(kn, d)
        assert np.allclose(S[h], Sh, rtol=1e-5, atol=1e-6)
        assert np.allclose(o[0, h], Sh.T @ qn, rtol=1e-4, atol=1e-5)
