"""The C ABI library builds, loads without a GPU, and exports every function
include/warp_hip.h declares; registration declines when there is no device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "warp_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = set(re.findall(r"\b((?:warp_hip|waste)_\w+)\s*\(", src))
    return sorted(n for n in names if not n.endswith("_fn"))


def test_header_declares_the_abi():
    names = declared()
    for must in ("waste_register_hip", "warp_hip_open", "warp_hip_moe_decode", "warp_hip_moe_chunk",
                 "warp_hip_vq_matvec", "warp_hip_decode_weights", "warp_hip_route"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import warp_amd
    L = warp_amd.lib()
    missing = [n for n in declared() if not hasattr(L, n)]
    assert not missing, missing
    from warp_amd import hip
    assert set(declared()) <= set(hip.SIGNATURES)


def test_registration_declines_without_a_device():
    import warp_amd
    from warp_amd.device import device_count
    if device_count() > 0:
        pytest.skip("a device is present")

    class Table(ctypes.Structure):
        _fields_ = [("fn", ctypes.c_void_p * 5), ("on_device", ctypes.c_int)]

    t = Table()
    t.fn[3] = 1234
    assert warp_amd.lib().waste_register_hip(ctypes.byref(t)) is None
    assert t.fn[3] == 1234 and t.on_device == 0


def test_open_refuses_without_a_device():
    import warp_amd
    from warp_amd.device import device_count
    if device_count() > 0:
        pytest.skip("a device is present")
    with pytest.raises(warp_amd.WarpHipError):
        warp_amd.Context(hidden=128, inter=64, n_experts=8, top_k=2, n_layers=1, fmt="VQ3R",
                         rec_bytes=12288, cache_bytes=12288 * 8)
