"""warp_amd — MI355X (gfx950) backend for WARP's routed-expert MoE path.

The product is the C ABI in include/warp_hip.h, built into
warp_amd/libwarp_hip.so by warp_amd.build; warp_amd.hip binds it with ctypes.
"""
from .hip import Context, WarpHipError, lib, load_container_model  # noqa: F401

__all__ = ["Context", "WarpHipError", "lib", "load_container_model"]
