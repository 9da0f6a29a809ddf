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


# Wait states the compiler keeps between an MFMA and a VALU (or load) that reads or overwrites its
# result in straight-line code on gfx950, the least over every decode kernel's straight-line pairs
# (hipcc of ROCm 7.2): 8 after v_mfma_f32_16x16x32_f16, 10 after v_mfma_f32_16x16x4_f32.
MFMA_WAIT = {"v_mfma_f32_16x16x32_f16": 8, "v_mfma_f32_16x16x4_f32": 10}


def _vregs(tok: str) -> set[int]:
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", tok):
        out.update([int(m.group(3))] if m.group(3) else range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def mfma_short_paths(lines: list[str]) -> list[tuple[int, str, int, str]]:
    """(wait states, MFMA, index, instruction) for every VALU or load that reads or overwrites an MFMA's
    destination registers within fewer wait states than MFMA_WAIT on some path of the control-flow graph
    (branch targets and fall-throughs alike; s_nop N counts N + 1, any other instruction 1)."""
    ins, labels = [], {}
    for l in lines:
        if re.match(r"^\.LBB\d+_\d+:$", l):
            labels[l[:-1]] = len(ins)
        elif l and not l.startswith("."):
            ins.append(l)

    def succ(k):
        t = ins[k]
        tgt = re.search(r"(\.LBB\d+_\d+)", t)
        if t.startswith("s_branch"):
            return [labels[tgt.group(1)]]
        if t.startswith("s_cbranch"):
            return [labels[tgt.group(1)], k + 1]
        if t.startswith(("s_endpgm", "s_setpc")):
            return []
        return [k + 1]

    def rw(t):
        op, _, rest = t.partition(" ")
        ops = [o.strip() for o in rest.split(",")] if rest else []
        if not ops or op.startswith("s_") or t.endswith(" lds"):
            return set(), set()
        if op.startswith(("global_store", "buffer_store", "ds_write", "scratch_store")):
            return _vregs(rest), set()
        r = _vregs(",".join(ops[1:])) | (_vregs(ops[0]) if op.startswith(("v_fmac", "v_mac")) else set())
        return r, _vregs(ops[0])

    found = {}
    for p, t in enumerate(ins):
        op = t.split()[0]
        if not op.startswith("v_mfma"):
            continue
        need = MFMA_WAIT.get(op, 8)
        dst = _vregs(t.split(None, 1)[1].split(",")[0])
        stack, seen = [(q, dst, 0) for q in succ(p)], set()
        while stack:
            k, live, w = stack.pop()
            if k >= len(ins) or not live or w >= need or (k, frozenset(live), w) in seen:
                continue
            seen.add((k, frozenset(live), w))
            u = ins[k]
            uop = u.split()[0]
            r, wr = rw(u)
            if uop.startswith("v_mfma"):
                live = live - _vregs(u.split(None, 1)[1].split(",")[0])   # a newer MFMA owns them
            elif (r | wr) & live:
                found[(p, k)] = min(found.get((p, k), need), w)
                live = live - wr
            nw = w + (int(u.split()[1]) + 1 if uop == "s_nop" else 1)
            stack.extend((q, live, nw) for q in succ(k))
    return sorted((w, ins[p], k, ins[k]) for (p, k), w in found.items())


def test_mfma_hazard_checker_finds_a_short_branch_path():
    """The checker on a hand-written case: the read of an MFMA result after a branch whose taken path
    skips the block that holds the wait states (a uniform branch over a masking block, as the
    one-stream page step once compiled) is flagged; with the wait states before the branch it is not."""
    bad = ["v_mfma_f32_16x16x32_f16 v[74:77], v[128:131], v[30:33], v[98:101]", "s_cbranch_scc1 .LBB0_2",
           "s_nop 7", "v_mov_b32_e32 v97, 0xff800000", ".LBB0_2:", "s_min_i32 s8, s99, 0x3fe",
           "v_fmamk_f32 v11, v76, 0xc1000000, v74", "s_endpgm"]
    hits = mfma_short_paths(bad)
    assert [(w, u) for w, _, _, u in hits] == [(2, "v_fmamk_f32 v11, v76, 0xc1000000, v74")]
    good = bad[:1] + ["s_nop 7"] + bad[1:]
    assert mfma_short_paths(good) == []
    straight = ["v_mfma_f32_16x16x4_f32 v[2:5], v1, v12, v[2:5]", "s_nop 7", "v_mov_b32_e32 v3, v9", "s_endpgm"]
    assert [w for w, *_ in mfma_short_paths(straight)] == [8]          # 10 needed after the fp32 MFMA


def test_mfma_results_keep_their_wait_states_on_every_path(asm):
    """Every VALU or load that reads or overwrites an MFMA result waits the compiler's own straight-line
    distance on every path, branch joins included. The compiler's hazard check does not cover a join
    reached by a taken branch from before the block that holds its wait states: a one-stream page step
    once read the scale half of its last bias MFMA 3 wait states after it on that path, and the page's
    scores lost their -HALF sum ks q' term whenever the pair's second page was valid."""
    bad = {name: hits[:3] for name, lines in kernels(asm).items() if (hits := mfma_short_paths(lines))}
    assert not bad, bad
