"""The Kimi Delta Attention recurrence on the device against the compiled
reference's waste_kda_step (src/kda.c:26-68), whose outputs over several
steps and shapes are in tests/golden/kda.npz (make_kda.py), and against the
oracle's restatement on larger shapes.

- warp_hip_kda_forward: T steps in one launch, state in device memory: the
  state and every step's output bit for bit.
- The kda_step slot that waste_register_hip fills (host pointers, as the
  engine calls it): bit for bit, the device-call counter advances, and a
  call the device cannot take (V above 1024) falls back to the table's
  previous slot with the same arguments.
"""
import ctypes as C
import os

import numpy as np
import pytest

from gpu_util import dev, empty, host, log
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KDA = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                  C.c_void_p, C.c_void_p, C.c_void_p)


class Table(C.Structure):
    _fields_ = [("kda_step", C.c_void_p), ("short_conv_step", C.c_void_p), ("rmsnorm_gated", C.c_void_p),
                ("mvq_rows_f32", C.c_void_p), ("lutb_range", C.c_void_p), ("on_device", C.c_int)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def forward_dev(q, k, v, g, beta, S0):
    import warp_amd.hip as wh
    from warp_amd.device import synchronize
    T, H, K = q.shape
    V = v.shape[2]
    Sd = dev(np.ascontiguousarray(S0, np.float32))
    od = empty((T, H, V))
    args = [dev(np.ascontiguousarray(z, np.float32)) for z in (q, k, v, g, beta)]
    assert wh.lib().warp_hip_kda_forward(T, H, K, V, *(a.ptr for a in args), Sd.ptr, od.ptr, None) == 0
    synchronize()
    return host(Sd), host(od)


def test_kda_forward_against_the_reference():
    g = dict(np.load(os.path.join(HERE, "kda.npz")))
    for n in range(3):
        S, o = forward_dev(g[f"c{n}_q"], g[f"c{n}_k"], g[f"c{n}_v"], g[f"c{n}_g"], g[f"c{n}_beta"], g[f"c{n}_S0"])
        assert np.array_equal(bits(S), bits(g[f"c{n}_S"])), n
        assert np.array_equal(bits(o), bits(g[f"c{n}_o"])), n
    log("kda forward: state and outputs bit-identical to the reference's waste_kda_step on 3 shapes")


@pytest.mark.parametrize("T,H,K,V", [(4, 32, 128, 128), (2, 8, 256, 64), (1, 5, 72, 200)])
def test_kda_forward_against_the_oracle(T, H, K, V):
    rng = np.random.default_rng(T * 1000 + K + V)
    q, k = rng.normal(size=(T, H, K)), rng.normal(size=(T, H, K))
    v, gl = rng.normal(size=(T, H, V)), -rng.uniform(0, 3, size=(T, H, K))
    beta, S0 = rng.uniform(0, 1, size=(T, H)), rng.normal(size=(H, K, V)) * 0.1
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    Sr, orf = po.kda_forward(f32(q), f32(k), f32(v), f32(gl), f32(beta), f32(S0))
    S, o = forward_dev(q, k, v, gl, beta, S0)
    assert np.array_equal(bits(S), bits(Sr)) and np.array_equal(bits(o), bits(orf))
    log(f"kda forward T={T} H={H} K={K} V={V}: bit-identical to the oracle")


def test_kda_slot_through_the_table():
    import warp_amd
    calls = []

    def prev(H, K, V, *ptrs):
        calls.append((H, K, V))
    prev_cb = KDA(prev)
    t = Table()
    t.kda_step = C.cast(prev_cb, C.c_void_p).value
    assert warp_amd.lib().waste_register_hip(C.byref(t)) and t.on_device == 1
    slot = KDA(t.kda_step)
    stats = lambda: (lambda a, b: (warp_amd.lib().warp_hip_kda_stats(C.byref(a), C.byref(b)), (a.value, b.value))[1])(
        C.c_uint64(), C.c_uint64())
    g = dict(np.load(os.path.join(HERE, "kda.npz")))
    d0, f0 = stats()
    for n in range(3):
        T, H, K = g[f"c{n}_q"].shape
        V = g[f"c{n}_v"].shape[2]
        S = g[f"c{n}_S0"].copy()
        o = np.empty((T, H, V), np.float32)
        u = np.empty(V, np.float32)
        for s in range(T):
            a = [np.ascontiguousarray(g[f"c{n}_{z}"][s]) for z in ("q", "k", "v", "g", "beta")]
            slot(H, K, V, *(z.ctypes.data for z in a), S.ctypes.data, o[s].ctypes.data, u.ctypes.data)
        assert np.array_equal(bits(S), bits(g[f"c{n}_S"])) and np.array_equal(bits(o), bits(g[f"c{n}_o"])), n
    d1, f1 = stats()
    assert d1 - d0 == sum(g[f"c{n}_q"].shape[0] for n in range(3)) and f1 == f0 and not calls
    # the device refuses V > 1024: the previous slot runs instead
    big = np.zeros(2 * 2048, np.float32)
    slot(1, 2, 2048, *(big.ctypes.data for _ in range(5)), np.zeros(2 * 2048, np.float32).ctypes.data,
         big.ctypes.data, big.ctypes.data)
    assert calls == [(1, 2, 2048)] and stats()[1] == f0 + 1
    log("kda_step slot: bit-identical to the reference through the table; a refused call falls back")
