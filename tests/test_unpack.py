"""The packed-prefill unpack on the CPU: pins the oracle's kush_cpu_unpack (the reference's CPU
kernel, cpu.mojo:122-169, restated) and the host-side index checks of Ops.unpack.

Pins, each failing on a different plausible mistake:
- the reference test's own fp64 torch oracle (tests/test_cpu.py:458-477 over _ops.py:398-436),
  restated in _unpack_fixture.unpack_torch: nibble order, sign extension, which scale goes with
  which axis, the tail slot, the row placement, gap rows left alone;
- records built from chosen codes and exactly representable scales / biases, whose dequantized
  values are known in closed form (independent of the record decoder the restatement shares);
- rot == the plain unpack followed by the canonical rotation of every history row, with new rows
  never rotated (tests/test_cpu.py:515-528);
- the index checks reject each kind of bad index (tests/test_cpu.py:494-512)."""
import pytest
import torch

from _unpack_fixture import INDEX_NAMES, history_rows, make_group, unpack_torch
from kushkash_amd._ops import PAGE, check_unpack_indices, fwht_reference, record_bytes
from oracle.cpu_ops import OracleOps


def oracle_unpack(c: dict, D: int, bits: int, rot: bool):
    ops = OracleOps("cpu", D, bits, 1)
    shape = (c["rows"], c["H"], D)
    kp, vp = torch.full(shape, float("nan")), torch.full(shape, float("nan"))
    args = [c[n].float() if n in ("tail_k", "k_new", "v_new") else c[n] for n in INDEX_NAMES]
    ops.unpack(c["records"], *args, kp, vp, rot)
    return kp, vp


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rot", [False, True])
def test_oracle_unpack_matches_fp64_torch(D, bits, rot):
    c = make_group(D, bits, torch.float32, seed=D + bits)
    kp, vp = oracle_unpack(c, D, bits, rot)
    rk, rv = unpack_torch(c, D, bits, rot, torch.float32)
    for got, want in ((kp, rk), (vp, rv)):
        same = got.view(torch.int32) == want.view(torch.int32)
        assert same.all(), f"{(~same).sum().item()} of {same.numel()} values differ"
    gaps = torch.tensor(c["gaps"])
    assert kp[gaps].isnan().all() and vp[gaps].isnan().all()          # never written
    written = torch.ones(c["rows"], dtype=torch.bool)
    written[gaps] = False
    assert not kp[written].isnan().any() and not vp[written].isnan().any()


def _record_from_codes(kc, ks, kb, vc, vs, vb, D: int, bits: int) -> torch.Tensor:
    """One record [RB] from codes kc, vc [32, D] (int) and fp16 ks, kb [D], vs, vb [32]: the
    layout written out directly (int4: byte j of a row = dim j low nibble, dim j + D/2 high)."""
    def rows(c):
        c = c.to(torch.int32)
        if bits == 8:
            return (c & 0xFF).to(torch.uint8)
        return ((c[:, :D // 2] & 0xF) | ((c[:, D // 2:] & 0xF) << 4)).to(torch.uint8)
    meta = torch.cat([ks, kb, vs, vb]).half().view(torch.uint8)
    out = torch.cat([rows(kc).reshape(-1), rows(vc).reshape(-1), meta])
    assert out.numel() == record_bytes(D, bits)
    return out


@pytest.mark.parametrize("D,bits", [(64, 4), (128, 8), (256, 4)])
def test_oracle_unpack_known_answers(D, bits):
    """Codes spanning the whole signed range, scales powers of two, biases multiples of the scale:
    every dequantized value code * s + b is exact in fp32, so the expected rows are known."""
    half = 1 << (bits - 1)
    g = torch.Generator().manual_seed(D * bits)
    kc = torch.randint(-half, half, (PAGE, D), generator=g)
    vc = torch.randint(-half, half, (PAGE, D), generator=g)
    kc[0] = torch.arange(D) % (2 * half) - half                       # every code at least once
    ks = 2.0 ** torch.randint(-6, 2, (D,), generator=g).float()
    kb = torch.randint(-40, 40, (D,), generator=g).float() * ks
    vs = 2.0 ** torch.randint(-6, 2, (PAGE,), generator=g).float()
    vb = torch.randint(-40, 40, (PAGE,), generator=g).float() * vs
    rec = _record_from_codes(kc, ks, kb, vc, vs, vb, D, bits).view(1, 1, -1)
    i32 = lambda *x: torch.tensor(x, dtype=torch.int32)
    kp, vp = torch.zeros(PAGE, 1, D), torch.zeros(PAGE, 1, D)
    empty = torch.zeros(0, 1, D)
    OracleOps("cpu", D, bits, 1).unpack(rec, i32(0), i32(0), i32(), i32(), torch.zeros(1, 1, PAGE, D), empty, empty,
                                        i32(), kp, vp, False)
    assert torch.equal(kp[:, 0], kc.float() * ks + kb)
    assert torch.equal(vp[:, 0], vc.float() * vs[:, None] + vb[:, None])


def test_oracle_unpack_rot_is_rotating_back():
    D, bits = 128, 4
    c = make_group(D, bits, torch.float32, seed=3)
    k0, v0 = oracle_unpack(c, D, bits, False)
    k1, v1 = oracle_unpack(c, D, bits, True)
    hist = history_rows(c)
    assert torch.equal(k1[hist], fwht_reference(k0[hist]))
    assert torch.equal(v1[hist], fwht_reference(v0[hist]))
    new = c["new_dst"].long()
    assert torch.equal(k1[new], c["k_new"]) and torch.equal(v1[new], c["v_new"])   # new rows: not rotated


def test_unpack_index_checks():
    c = make_group(64, 4, torch.float32)
    rows, blocks, slots = c["rows"], c["records"].shape[0], c["tail_k"].shape[0]

    def check(**over):
        a = {n: over.get(n, c[n]) for n in ("page_blk", "page_dst", "tail_blk", "tail_info", "new_dst")}
        check_unpack_indices(**a, rows=rows, blocks=blocks, slots=slots)

    check()                                                           # the valid group passes
    i32 = lambda *x: torch.tensor(x, dtype=torch.int32)
    info = c["tail_info"]
    bad = {"page_dst": dict(page_dst=c["page_dst"] + rows), "new_dst": dict(new_dst=c["new_dst"] + rows),
           "page_blk": dict(page_blk=c["page_blk"] + blocks), "tail_blk": dict(tail_blk=c["tail_blk"] - blocks),
           "tail_info tokens": dict(tail_info=torch.cat([i32(int(info[0]), PAGE + 1, 0), info[3:]])),
           "tail_info slot": dict(tail_info=torch.cat([info[:3], i32(int(info[3]), int(info[4]), slots)]))}
    bad["tail_info rows"] = dict(tail_info=torch.cat([info[:6], i32(rows - 2, 3, int(info[8]))]))
    for name, over in bad.items():
        with pytest.raises(ValueError, match=name):
            check(**over)
