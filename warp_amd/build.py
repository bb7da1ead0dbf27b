"""Builds libwarp_hip.so in-tree: the gfx950 kernels with hipcc, the C host
backend with gcc against the HIP runtime headers, linked into one shared
library that exports the C ABI of include/warp_hip.h.

    python -m warp_amd.build          (or __graft_entry__.build())
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libwarp_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    # packed fp32 instructions are kept out of generated code on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]
C_FLAGS = ["-O2", "-std=gnu11", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
           "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include"]


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l
                    and "is not a recognized feature for this target" not in l)
    if out.strip():
        print(out)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}")


def build(verbose: bool = True) -> str:
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    os.makedirs(BUILD, exist_ok=True)
    inc = [f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}"]
    k_obj = os.path.join(BUILD, "kernels.o")
    b_obj = os.path.join(BUILD, "backend.o")
    e_obj = os.path.join(BUILD, "encode.o")
    n_obj = os.path.join(BUILD, "noalloc.o")
    c_obj = os.path.join(BUILD, "crc.o")
    d_obj = os.path.join(BUILD, "kda.o")
    m_obj = os.path.join(BUILD, "moe_table.o")
    _run([hipcc, *HIP_FLAGS, *inc, "-c", os.path.join(CSRC, "kernels.hip"), "-o", k_obj])
    _run([hipcc, *HIP_FLAGS, *inc, "-c", os.path.join(CSRC, "noalloc.hip"), "-o", n_obj])
    _run([hipcc, *HIP_FLAGS, *inc, "-c", os.path.join(CSRC, "crc.hip"), "-o", c_obj])
    _run([hipcc, *HIP_FLAGS, *inc, "-c", os.path.join(CSRC, "kda.hip"), "-o", d_obj])
    _run(["gcc", *C_FLAGS, *inc, "-c", os.path.join(CSRC, "backend.c"), "-o", b_obj])
    _run(["gcc", *C_FLAGS, *inc, "-c", os.path.join(CSRC, "encode.c"), "-o", e_obj])
    _run(["gcc", *C_FLAGS, *inc, "-c", os.path.join(CSRC, "moe_table.c"), "-o", m_obj])
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, k_obj, n_obj, c_obj, d_obj, b_obj, e_obj, m_obj,
          f"-L{ROCM}/lib", "-lamdhip64", "-lpthread", f"-Wl,-rpath,{ROCM}/lib",
          "-Wl,--no-undefined"])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
