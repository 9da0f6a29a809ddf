"""Ahead-of-time build of the gfx950 HIP library (replaces the reference's first-use Mojo build,
kushkash/_build.py:215-254): one hipcc invocation over csrc/*.hip into kushkash_amd/libkushhip.so.

    python -m kushkash_amd.build
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB = PKG / "libkushhip.so"
SOURCES = ("kush_capi.hip", "kush_write.hip", "kush_decode.hip", "kush_rotate.hip",
           "kush_unpack.hip")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-mcode-object-version=5",
    # quantization must divide like IEEE fp32 (bit-exact pages); never -ffast-math
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # no packed-fp32 VALU forms (v_pk_fma_f32 / v_pk_mul_f32 / v_pk_add_f32) anywhere
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the decode kernels then need no v_accvgpr moves in their page loop
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wno-pass-failed",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build kushkash_amd)")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 into LIB (always recompiles); returns the path."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, f"-I{ROOT / 'include'}", "-o", str(tmp), *(str(PKG / "csrc" / s) for s in SOURCES)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"          # host pass: harmless
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
