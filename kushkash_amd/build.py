"""Ahead-of-time build of the gfx950 HIP library (replaces the reference's first-use Mojo build,
kushkash/_build.py:215-254): csrc/*.hip compiled to objects in parallel (the decode instantiations
once per input dtype and rot flag), then linked into kushkash_amd/libkushhip.so; beside it the CPU
path's host library kushkash_amd/libkushcpu.so (csrc/kush_cpu.cpp, g++).

    python -m kushkash_amd.build
"""
from __future__ import annotations

import hashlib
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
DIGEST = PKG / "libkushhip.so.digest"          # source digest of the library last built here
# A profiling copy of the library: the same objects with the bf16 / rot 0 decode instantiations
# recompiled with -DKUSH_TIMELINE (per-workgroup phase timestamps and XCD ids, kush_decode.h), read by
# `python bench.py --timeline`. The product never loads it.
TIMELINE_LIB = PKG / "libkushhip_timeline.so"
# A measurement instrument beside the product: the decode's streaming floor (csrc/kush_floor.hip, the
# same records, launch shape and DMA ring as the decode without its math), loaded only by bench.py.
FLOOR_LIB = PKG / "libkushfloor.so"
FLOOR_SOURCE = "kush_floor.hip"
# The host library of the package's CPU path (csrc/kush_cpu.cpp, g++ with OpenMP): Ops and KushCache on
# device "cpu", the reference's CPU library's C ABI (kushkash/_cpu.py).
CPU_LIB = PKG / "libkushcpu.so"
CPU_SOURCE = "kush_cpu.cpp"
CPU_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off"]
SOURCES = ("kush_capi.hip", "kush_write.hip", "kush_decode.hip", "kush_rotate.hip",
           "kush_unpack.hip", "kush_decode_inst.hip")
# the decode kernel instantiations: one object per (input dtype, rot)
DECODE_INST = [{"KUSH_INST_IN": t, "KUSH_INST_ROT": r} for t in ("float", "_Float16", "kush::bf16_t") for r in (0, 1)]


TIMELINE_UNIT = ("kush_decode_inst.hip", {"KUSH_INST_IN": "kush::bf16_t", "KUSH_INST_ROT": 0})


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


def _includes(path: Path, seen: set) -> None:
    """path and the local headers it includes, transitively (csrc/ and include/)."""
    import re
    if path in seen or not path.exists():
        return
    seen.add(path)
    for name in re.findall(r'^\s*#\s*include\s+"([^"]+)"', path.read_text(), re.M):
        for d in (path.parent, PKG / "csrc", ROOT / "include"):
            if (d / name).exists():
                _includes(d / name, seen)
                break


def _code(text: str) -> str:
    """C / C++ source without its comments, blank lines and indentation (spaces inside a line
    collapsed; line breaks kept, as they end preprocessor directives): what the compiler reads
    (string and character literals are kept as they are)."""
    out, i, n = [], 0, len(text)
    while i < n:
        ch = text[i]
        if ch in "\"'":
            j = i + 1
            while j < n and text[j] != ch:
                j += 2 if text[j] == "\\" else 1
            out.append(text[i:j + 1])
            i = j + 1
        elif text.startswith("//", i):
            while i < n and text[i] != "\n":
                i += 1
        elif text.startswith("/*", i):
            j = text.find("*/", i + 2)
            i = n if j < 0 else j + 2
            out.append(" ")
        else:
            out.append(ch)
            i += 1
    lines = (" ".join(line.split()) for line in "".join(out).splitlines())
    return "\n".join(line for line in lines if line)


def source_digest(unit: str | None = None) -> str:
    """16 hex digits of sha256 over what decides the machine code of one translation unit (`unit`, a
    csrc/*.hip file: it and its local headers, transitively) or of the whole library (None: every
    source and header) -- their code without comments or layout -- plus the compiler flags and
    instantiation units. The same code gives the same digest on every machine and rebuild, so a
    measurement of a kernel taken on one build can be matched to the build that runs later, and stays
    valid while only other kernels or comments change."""
    h = hashlib.sha256()
    if unit is None:
        files = sorted((PKG / "csrc").glob("*.h")) + sorted((PKG / "csrc").glob("*.hip"))
        files.append(ROOT / "include" / "kushkash_amd.h")
    else:
        seen: set = set()
        _includes(PKG / "csrc" / unit, seen)
        files = sorted(seen)
    for f in files:
        h.update(f.name.encode() + b"\0" + _code(f.read_text()).encode() + b"\0")
    h.update(repr(CPU_FLAGS if unit == CPU_SOURCE else (FLAGS, units())).encode())
    return h.hexdigest()[:16]


def built_digest(unit: str | None = None) -> str | None:
    """The source digest (of `unit`, or of the whole library) recorded when LIB was built, or None if
    LIB was not built by build()."""
    import json
    try:
        return json.loads(DIGEST.read_text()).get(unit or "all")
    except (OSError, ValueError):
        return None


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
        raise RuntimeError(f"{Path(cmd[0]).name} failed ({res.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def cxx() -> str:
    for cand in (os.environ.get("CXX"), shutil.which("g++"), "/usr/bin/g++"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("g++ not found (the CPU path's library is built with it)")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 into LIB, TIMELINE_LIB from the same objects with the
    timeline unit instrumented, the measurement library FLOOR_LIB, and the CPU path's host library
    CPU_LIB (always recompiles; objects in parallel, then the links); returns LIB."""
    todo = units() + [(FLOOR_SOURCE, {}), (TIMELINE_UNIT[0], dict(TIMELINE_UNIT[1], KUSH_TIMELINE=1))]
    jobs = jobs or max(1, min(len(todo), int(os.environ.get("MAX_JOBS", 0)) or os.cpu_count() or 1))
    compile_flags = [f for f in FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="kushkash_amd_build_") as tmpdir:
        objs, cmds = [], []
        for i, (src, defs) in enumerate(todo):
            obj = str(Path(tmpdir) / f"{i:02d}_{Path(src).stem}.o")
            objs.append(obj)
            cmds.append([hipcc(), *compile_flags, *(f"-D{k}={v}" for k, v in defs.items()), f"-I{ROOT / 'include'}",
                         "-c", str(PKG / "csrc" / src), "-o", obj])
        cpu_tmp = CPU_LIB.with_suffix(".so.tmp")
        cmds.append([cxx(), *CPU_FLAGS, f"-I{ROOT / 'include'}", "-o", str(cpu_tmp), str(PKG / "csrc" / CPU_SOURCE)])
        with ThreadPoolExecutor(jobs) as ex:
            list(ex.map(lambda c: _run(c, verbose), cmds))
        os.replace(cpu_tmp, CPU_LIB)
        product = objs[:len(units())]
        swap = units().index(TIMELINE_UNIT)
        timeline = product[:swap] + objs[-1:] + product[swap + 1:]
        for dst, parts in ((LIB, product), (TIMELINE_LIB, timeline), (FLOOR_LIB, objs[-2:-1])):
            tmp = dst.with_suffix(".so.tmp")
            _run([hipcc(), *FLAGS, "-o", str(tmp), *parts], verbose)
            os.replace(tmp, dst)
    import json
    DIGEST.write_text(json.dumps({"all": source_digest(),
                                  **{u: source_digest(u) for u in SOURCES + (FLOOR_SOURCE, CPU_SOURCE)}},
                                 indent=1) + "\n")
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
