"""The reference's dispatch-table slot on the device.

waste_register_hip fills mvq_rows_f32 in a waste_kernels table laid out as
src/waste_backend.h:67-90 and sets on_device; the engine then calls the
slot as run_rows(out, 64, waste_k.mvq_rows_f32, &a) with an mvq_arg of host
pointers (src/model.c:385-399, src/simd.h:35-39): the whole row range in
one call when on_device, 64-row pieces from pool threads otherwise. Here
the slot is called exactly that way for Q8G, Q4G and Q3G rows (3-bit rows
are a bitstream plus a guard byte, src/model.c:605-609), groups of 32, 64
and 128 with a ragged last group, over the whole range and over pieces.
Bar: within the fp32 summation bound of float64 against the oracle's
AVX-512 restatement of waste_mvq_rows_f32 (src/simd_avx512.c:20-88); the
device-call counter advances, and a call the device refuses (an
unsupported bit width) falls back to the table's previous slot with the
same arguments (src/metal.m:177-181).
"""
import ctypes as C

import numpy as np
import pytest

from gpu_util import log
from oracle import pyoracle as po

pytestmark = pytest.mark.gpu
SLOT = C.CFUNCTYPE(None, C.c_int, C.c_int, C.c_void_p)


class MvqArg(C.Structure):
    _fields_ = [("y", C.c_void_p), ("W", C.c_void_p), ("ws", C.c_void_p), ("xq", C.c_void_p),
                ("xs", C.c_void_p), ("in_", C.c_int), ("ng", C.c_int), ("group", C.c_int), ("bits", C.c_int),
                ("rowbytes", C.c_size_t)]


class Table(C.Structure):
    _fields_ = [("kda_step", C.c_void_p), ("short_conv_step", C.c_void_p), ("rmsnorm_gated", C.c_void_p),
                ("mvq_rows_f32", C.c_void_p), ("lutb_range", C.c_void_p), ("on_device", C.c_int)]


def quant_rows(rng, rows, n, bits, group):
    """Payload, fp16 scales, rowbytes and the float64 weights they stand for."""
    ng = (n + group - 1) // group
    q = rng.integers(-(1 << (bits - 1)) + (bits == 8), 1 << (bits - 1), size=(rows, ng * group))
    if bits == 8:
        rowbytes = ng * group
        pay = (q & 0xFF).astype(np.uint8)
    elif bits == 4:
        rowbytes = ng * group // 2
        pay = ((q[:, 0::2] + 8) | ((q[:, 1::2] + 8) << 4)).astype(np.uint8)
    else:
        rowbytes = (ng * group * 3 + 7) // 8 + 1
        pay = np.zeros((rows, rowbytes), np.uint8)
        u = (q + 4).astype(np.uint32)
        for i in range(ng * group):
            off = 3 * i
            pay[:, off >> 3] |= ((u[:, i] << (off & 7)) & 0xFF).astype(np.uint8)
            pay[:, (off >> 3) + 1] |= ((u[:, i] << (off & 7)) >> 8).astype(np.uint8)
    sc = rng.uniform(0.002, 0.02, size=(rows, ng)).astype(np.float16)
    Wf = q.astype(np.float64) * np.repeat(sc.astype(np.float64), group, axis=1)
    return np.ascontiguousarray(pay), sc.view(np.uint16).copy(), rowbytes, Wf[:, :n]


@pytest.fixture(scope="module")
def table():
    import warp_amd
    calls = []

    def prev(b, e, p):
        calls.append((b, e))
    prev_cb = SLOT(prev)
    t = Table()
    t.mvq_rows_f32 = C.cast(prev_cb, C.c_void_p).value
    name = warp_amd.lib().waste_register_hip(C.byref(t))
    assert name and name.decode().startswith("HIP") and t.on_device == 1
    assert t.mvq_rows_f32 != C.cast(prev_cb, C.c_void_p).value
    yield t, calls, prev_cb
    warp_amd.lib().waste_hip_release_host_buffers()


def stats():
    import warp_amd
    d, f = C.c_uint64(), C.c_uint64()
    warp_amd.lib().warp_hip_table_stats(C.byref(d), C.byref(f))
    return d.value, f.value


@pytest.mark.parametrize("bits,group,rows,n", [(8, 32, 256, 2304), (8, 64, 200, 1000), (4, 128, 384, 7168),
                                               (4, 32, 100, 333), (3, 64, 160, 2304), (3, 32, 96, 250)])
def test_mvq_slot_through_the_table(table, bits, group, rows, n):
    t, calls, _ = table
    rng = np.random.default_rng(bits * 1000 + group + n)
    pay, sc, rowbytes, Wf = quant_rows(rng, rows, n, bits, group)
    x = rng.standard_normal(n).astype(np.float32)
    ng = (n + group - 1) // group
    ref = np.empty(rows, np.float32)
    po.lib().or_mvq_rows_f32(0, rows, ref.ctypes.data, pay.ctypes.data, sc.ctypes.data, x.ctypes.data, n, ng,
                             group, bits, rowbytes, 2)
    exact = Wf @ x.astype(np.float64)
    bound = 2 * n * 2.0 ** -24 * (np.abs(Wf) @ np.abs(x).astype(np.float64))
    assert np.all(np.abs(ref - exact) <= bound), "the rows built here do not match the oracle's reading"
    slot = SLOT(t.mvq_rows_f32)
    d0, f0 = stats()
    n_calls = len(calls)
    for pieces in ([(0, rows)], [(b, min(b + 64, rows)) for b in range(0, rows, 64)]):
        y = np.full(rows, np.nan, np.float32)
        a = MvqArg(y.ctypes.data, pay.ctypes.data, sc.ctypes.data, None, x.ctypes.data, n, ng, group, bits,
                   rowbytes)
        for b, e in pieces:
            slot(b, e, C.cast(C.pointer(a), C.c_void_p))
        assert np.all(np.abs(y - exact) <= bound), float(np.max(np.abs(y - exact) / bound))
        assert np.all(np.abs(y - ref) <= bound)
    d1, f1 = stats()
    # the device mirrors are keyed by host address (trunk tensors outlive a
    # model's calls); these arrays do not, so drop them before they go
    import warp_amd
    warp_amd.lib().waste_hip_release_host_buffers()
    assert d1 - d0 == 1 + (rows + 63) // 64 and f1 == f0 and len(calls) == n_calls
    log(f"table slot Q{bits}G group {group}, {rows}x{n}: within the bound on the device "
        f"(max |d|/bound {float(np.max(np.abs(y - exact) / bound)):.3f})")


def test_refused_call_falls_back_to_the_previous_slot(table):
    t, calls, _ = table
    rng = np.random.default_rng(9)
    pay, sc, rowbytes, _ = quant_rows(rng, 64, 64, 8, 32)
    x = rng.standard_normal(64).astype(np.float32)
    y = np.zeros(64, np.float32)
    a = MvqArg(y.ctypes.data, pay.ctypes.data, sc.ctypes.data, None, x.ctypes.data, 64, 2, 32, 5, rowbytes)
    d0, f0 = stats()
    SLOT(t.mvq_rows_f32)(0, 64, C.cast(C.pointer(a), C.c_void_p))
    d1, f1 = stats()
    import warp_amd
    warp_amd.lib().waste_hip_release_host_buffers()
    assert calls and calls[-1] == (0, 64) and f1 == f0 + 1 and d1 == d0
    log("table slot: a refused device call ran the previous slot with the same arguments")
