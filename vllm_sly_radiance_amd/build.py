"""Build libw4a8_mxfp4.so in-tree with hipcc for gfx950 (one code object, no other target).

    python -m vllm_sly_radiance_amd.build            # or __graft_entry__.build()

The library is a plain C-ABI shared object (include/w4a8_mxfp4.h) loaded through ctypes; it links
the HIP runtime by soname, so inside a torch process it binds to the runtime torch already loaded.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libw4a8_mxfp4.so"
LIB_PATH = os.path.join(PKG, LIB_NAME)
ARCH = "gfx950"

SOURCES = ["w4a8_api.hip", "w4a8_quant.hip", "w4a8_repack.hip", "w4a8_gemm_skinny.hip",
           "w4a8_gemm_stream.hip", "w4a8_gemm_ring.hip", "w4a8_gemm_tile.hip", "w4a8_gemm_band.hip",
           "w4a8_producers.hip", "w4a8_probe.hip"]

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
    # keep the compiler from forming packed-fp32 VALU ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the first 14 kernel-argument dwords arrive in SGPRs at wave launch instead of through a
    # scalar load from the kernarg segment (the kernels order their arguments so that everything
    # the first memory requests depend on comes first); the code object keeps a 256-byte prologue
    # that loads them itself where the firmware does not preload
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def build(verbose: bool = False) -> str:
    """Compile every source into LIB_PATH (always rebuilds) and return the path."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is expected
    noise = [ln for ln in (res.stdout + res.stderr).splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln and "warning generated" not in ln
             and "warnings generated" not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(noise))
    if verbose and noise:
        print("\n".join(noise), file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
