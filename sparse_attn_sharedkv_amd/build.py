"""Build recipe for the HIP library (gfx950).

Compiles ``csrc/*.hip`` and ``csrc/*.cpp`` with ``hipcc`` into
``_lib/libsas_mi355x.so`` inside the package, so the built library travels
with the source tree. Run ``python -m sparse_attn_sharedkv_amd.build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_DIR = os.path.join(PKG, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libsas_mi355x.so")
SOURCES = [os.path.join(PKG, "csrc", n) for n in ("sas_attn.hip", "sas_kv_fp8.hip", "sas_metadata.cpp",
                                                   "sas_metadata_dev.hip")]
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed FP32 VALU forms are kept out of generated code on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the online-softmax rescale multiplies them with
    # VALU ops, which cannot read AGPRs (AGPR-resident accumulators cost a full
    # copy out and back on every tile)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found (ROCm is required to build the library)")
    return exe


def build(verbose: bool = False) -> str:
    """Compile the library; returns its path. Always recompiles."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIP_FLAGS, "-x", "hip", *SOURCES, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    if verbose:
        sys.stdout.write(res.stdout)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
