"""Ahead-of-time build of the gfx950 HIP library (replaces the reference's first-use Mojo build,
kushkash/_build.py:215-254): csrc/*.hip compiled to objects in parallel (the decode instantiations
once per input dtype and rot flag), then linked into kushkash_amd/libkushhip.so.

    python -m kushkash_amd.build
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB = PKG / "libkushhip.so"
SOURCES = ("kush_capi.hip", "kush_write.hip", "kush_decode.hip", "kush_rotate.hip",
           "kush_unpack.hip", "kush_decode_inst.hip")
# the decode kernel instantiations: one object per (input dtype, rot)
DECODE_INST = [{"KUSH_INST_IN": t, "KUSH_INST_ROT": r} for t in ("float", "_Float16", "kush::bf16_t") for r in (0, 1)]


def units() -> list[tuple[str, dict]]:
    """(source, preprocessor defines) of every object of the library."""
    out = []
    for s in SOURCES:
        out += [(s, d) for d in DECODE_INST] if s == "kush_decode_inst.hip" else [(s, {})]
    return out
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


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"          # host pass: harmless
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 into LIB (always recompiles; objects in parallel, then one
    link); returns the path."""
    jobs = jobs or max(1, min(len(units()), int(os.environ.get("MAX_JOBS", 0)) or os.cpu_count() or 1))
    compile_flags = [f for f in FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="kushkash_amd_build_") as tmpdir:
        objs, cmds = [], []
        for i, (src, defs) in enumerate(units()):
            obj = str(Path(tmpdir) / f"{i:02d}_{Path(src).stem}.o")
            objs.append(obj)
            cmds.append([hipcc(), *compile_flags, *(f"-D{k}={v}" for k, v in defs.items()), f"-I{ROOT / 'include'}",
                         "-c", str(PKG / "csrc" / src), "-o", obj])
        with ThreadPoolExecutor(jobs) as ex:
            list(ex.map(lambda c: _run(c, verbose), cmds))
        tmp = LIB.with_suffix(".so.tmp")
        _run([hipcc(), *FLAGS, "-o", str(tmp), *objs], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
