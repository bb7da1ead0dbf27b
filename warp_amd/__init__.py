"""warp_amd — MI355X (gfx950) backend for WARP's routed-expert MoE path.

The product is the C ABI in include/warp_hip.h, built into
warp_amd/libwarp_hip.so by warp_amd.build; warp_amd.hip binds it with ctypes.
"""
from .hip import (E_ARG, E_BOOKS, E_CRC, E_DEVICE, E_HEADER, E_MISSING, E_NOMEM, E_NOSLOT,  # noqa: F401
                  E_READ, Context, WarpHipError, lib, load_container_model)

__all__ = ["Context", "WarpHipError", "lib", "load_container_model", "E_ARG", "E_DEVICE", "E_NOMEM", "E_READ",
           "E_HEADER", "E_CRC", "E_NOSLOT", "E_MISSING", "E_BOOKS"]
