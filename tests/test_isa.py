"""Static checks of the decode kernels' gfx950 assembly (hipcc -S, on the CPU).

The page loop issues its buffer-to-LDS loads in asm, out of the compiler's sight, and waits for
them with explicit vmcnt counts; the asm sets m0, which the compiler reserves. That is sound only
while (1) nothing else in these kernels reads m0 (no movrel / gpr-index instructions, every write
of m0 is the one our load sequence makes), (2) each m0 write is separated from the LDS DMA that
reads it by one wait state (the compiler's own LDS DMAs keep that distance; it cannot add it inside
the asm) and (3) the compiler inserts no LDS-DMA of its own."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "kushkash_amd" / "csrc" / "kush_decode_inst.hip"


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    """The device assembly of every decode instantiation: one compile per (input dtype, rot), as the build."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    from concurrent.futures import ThreadPoolExecutor
    from kushkash_amd.build import DECODE_INST, FLAGS
    tmp = tmp_path_factory.mktemp("isa")
    flags = [f for f in FLAGS if f not in ("-shared", "-fPIC")]

    def compile_one(i_defs):
        i, defs = i_defs
        out = tmp / f"kush_decode_{i}.s"
        subprocess.run([hipcc, *flags, *(f"-D{k}={v}" for k, v in defs.items()), f"-I{ROOT / 'include'}", "-S",
                        "--cuda-device-only", str(SRC), "-o", str(out)], check=True, capture_output=True)
        return out.read_text()

    with ThreadPoolExecutor(len(DECODE_INST)) as ex:
        return "\n".join(ex.map(compile_one, enumerate(DECODE_INST)))


def kernels(asm_text: str) -> dict[str, list[str]]:
    """kernel symbol -> its instruction lines (decode kernels only)."""
    out, cur = {}, None
    for line in asm_text.splitlines():
        m = re.match(r"^(_ZN4kush13decode_kernel\w+):", line)
        if m:
            cur = m.group(1)
            out[cur] = []
        elif cur and re.match(r"^\s*\.Lfunc_end", line):
            cur = None
        elif cur:
            out[cur].append(line.split(";")[0].strip())
    return out


def test_m0_is_only_the_lds_load_base(asm):
    ks = kernels(asm)
    assert len(ks) >= 30, "expected every decode kernel instantiation"
    for name, lines in ks.items():
        for i, ins in enumerate(lines):
            assert not re.match(r"(v_movrel|s_movrel|s_set_gpr_idx|v_interp|ds_gws|s_sendmsg)", ins), (name, ins)
            if "m0" in ins:
                assert re.match(r"s_mov_b32 m0, s\d+$", ins), (name, ins)
                # one wait state between the m0 write and the LDS DMA that reads it, then the DMA
                nxt = [l for l in lines[i + 1:i + 4] if l]
                assert nxt[0] == "s_nop 0", (name, nxt[0])
                assert re.match(r"buffer_load_dwordx4 v\d+, s\[\d+:\d+\], 0 offen lds$", nxt[1]), (name, nxt[1])


def test_every_lds_load_is_ours(asm):
    for name, lines in kernels(asm).items():
        for i, ins in enumerate(lines):
            if ins.endswith(" lds") or "_lds_" in ins:
                prev = [l for l in lines[:i] if l][-2:]
                assert prev[0].startswith("s_mov_b32 m0,") and prev[1] == "s_nop 0", (name, prev, ins)


def test_split_merge_is_device_scope_accesses_without_cache_maintenance(asm):
    """The fused split-K merge communicates only through device-scope accesses: partials stored
    write-through (`global_store ... sc1`), one returning atomic add per workgroup on the split
    counter, partials read back past the local L2 (`global_load ... sc1`), and no L2 write-back or
    invalidate anywhere (no `buffer_wbl2` / `buffer_inv`, which a release / acquire would add)."""
    for name, lines in kernels(asm).items():
        assert not [l for l in lines if re.match(r"(buffer_wbl2|buffer_inv|buffer_wbinvl1)", l)], name
        atomics = [l for l in lines if l.startswith("global_atomic")]
        assert atomics, name                                        # every variant carries the merge
        for a in atomics:
            assert re.match(r"global_atomic_add v\d+, v\d+, v\d+, s\[\d+:\d+\] sc0$", a), (name, a)
        assert any(l.startswith("global_store") and l.endswith(" sc1") for l in lines), name
        assert any(l.startswith("global_load") and l.endswith(" sc1") for l in lines), name
