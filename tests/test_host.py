"""Host-side helpers of kushkash_amd on the CPU (no kernels): the Hadamard rotation
(tests/test_cpu.py:257-297 of the reference), the canonical FWHT order (_ops.py:380-395) checked
against the dense product and against the oracle's kush_cpu_fwht bit for bit, the log-sum-exp merge
of attention partials (_ops.py:279-285), token-major dequantization (tests/test_cpu.py:300-316),
page bookkeeping and the rotation switch."""
import math

import pytest
import torch

from kushkash_amd._ops import (FWHT_SCALE_BITS, PAGE, attn_lse, dequant_records, fwht_reference, hadamard, merge,
                               pages_touched, record_bytes, rotate, rotation_enabled)


def test_hadamard_is_orthonormal_and_symmetric():
    for D in (64, 128, 256):
        h = hadamard(D, "cpu").double()
        assert torch.allclose(h, h.T) and torch.allclose(h @ h, torch.eye(D, dtype=torch.float64), atol=1e-6)
        assert bool((h.abs() == torch.tensor(1 / math.sqrt(D), dtype=torch.float32).double()).all())


def test_hadamard_sylvester_order():
    """H_2n = [[H_n, H_n], [H_n, -H_n]] / sqrt(2) (Sylvester), the order of the reference's matrix."""
    for D in (64, 128, 256):
        h = torch.sign(hadamard(D, "cpu"))
        hn = torch.sign(hadamard(D // 2, "cpu"))
        assert torch.equal(h, torch.cat([torch.cat([hn, hn], 1), torch.cat([hn, -hn], 1)], 0))


def test_rotate_rounds_once():
    """rotate() = the exact orthonormal product rounded once into the output dtype, for strided inputs
    too; rotating twice gives x back; out= writes in place and rejects wrong sizes and aliasing."""
    unit = {torch.float32: 2.0 ** -24, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}
    torch.manual_seed(0)
    for dt, u in unit.items():
        for D in (64, 128, 256):
            h = hadamard(D, "cpu")
            x = torch.randn(6, 8, D).to(dt)[:, ::2]
            y = rotate(x, h)
            ref = x.double() @ h.double()
            assert y.dtype == dt and y.shape == x.shape and y.is_contiguous()
            assert bool(((y.double() - ref).abs() <= u * ref.abs() + 1e-5).all()), (dt, D)
            back = rotate(y, h).double()
            assert float((back - x.double()).norm() / x.double().norm()) < 2 * u * 4, (dt, D)
            assert rotate(x, None) is x and rotate(x, h, torch.float32).dtype == torch.float32
            buf = torch.full((8, 4, D), float("nan"), dtype=dt)
            rotate(x, h, out=buf[:6])
            assert torch.equal(buf[:6], y) and bool(buf[6:].isnan().all()), (dt, D)
            with pytest.raises(ValueError):
                rotate(x, h, out=buf[:3])
            with pytest.raises(ValueError):
                rotate(buf[:6], h, out=buf[1:7])


@pytest.mark.parametrize("D", [64, 128, 256])
def test_fwht_reference(D):
    """The canonical butterfly order equals the dense Hadamard product (fp64 check, fp32 rounding),
    its scale is fp32 1/sqrt(D), and the oracle's kush_cpu_fwht reproduces it bit for bit."""
    from oracle.cpu_ops import OracleOps
    torch.manual_seed(D)
    x = torch.randn(37, D)
    y = fwht_reference(x)
    dense = x.double() @ hadamard(D, "cpu").double()
    assert torch.allclose(y.double(), dense, rtol=1e-5, atol=1e-5)
    s = torch.tensor([FWHT_SCALE_BITS[D]], dtype=torch.int32).view(torch.float32)
    assert float(s) == pytest.approx(1 / math.sqrt(D), rel=1e-7)
    assert torch.equal(OracleOps("cpu", D, 4, 1).fwht(x.contiguous()), y)


def test_lse_merge_identity():
    """Attention over disjoint key blocks merged by log-sum-exp == attention over all keys."""
    torch.manual_seed(0)
    q = torch.randn(2, 6, 3, 64)
    k, v = torch.randn(2, 2, 100, 64), torch.randn(2, 2, 100, 64)
    full = attn_lse(q, k, v, False, 0.125)
    acc = None
    for a, b in ((0, 7), (7, 40), (40, 41), (41, 100)):
        acc = merge(acc, attn_lse(q, k[:, :, a:b], v[:, :, a:b], False, 0.125))
    assert torch.allclose(acc[0], full[0], atol=1e-5) and torch.allclose(acc[1], full[1], atol=1e-5)


def test_fused_refusal_falls_back_to_bounded_products(monkeypatch):
    """attn_lse(fused=True) when the flash kernel refuses a block it was told to take: the fp32 products
    over key sub-blocks sized for their scores, merged by log-sum-exp, the same as one product."""
    from kushkash_amd import _attention as A
    monkeypatch.setattr(A, "fused_ok", lambda q: True)
    monkeypatch.setattr(A, "_flash", lambda *a, **k: None)
    monkeypatch.setattr(A, "keys_per_block", lambda *a, **k: 16)            # force several sub-blocks
    torch.manual_seed(1)
    q = torch.randn(2, 6, 3, 64)
    k, v = torch.randn(2, 2, 100, 64), torch.randn(2, 2, 100, 64)
    out, lse = A.attn_lse(q, k, v, False, 0.125, fused=True)
    ref_out, ref_lse = A.attn_lse(q, k, v, False, 0.125)
    assert torch.allclose(out, ref_out, atol=1e-5) and torch.allclose(lse, ref_lse, atol=1e-5)


@pytest.mark.parametrize("bits", [4, 8])
def test_dequant_token_major(bits):
    """token_major=True = the default layout with page and head axes swapped, contiguous."""
    for D in (64, 128, 256):
        for dt in (torch.float32, torch.bfloat16, torch.float16):
            rb, o = record_bytes(D, bits), 2 * PAGE * (D if bits == 8 else D // 2)
            rec = torch.randint(0, 256, (5, 3, rb), dtype=torch.uint8)
            rec[..., o:] = torch.randn(5, 3, (rb - o) // 2).half().view(torch.uint8)
            k, v = dequant_records(rec, D, bits, dt)
            kt, vt = dequant_records(rec, D, bits, dt, token_major=True)
            assert kt.is_contiguous() and vt.is_contiguous()
            assert torch.equal(kt, k.transpose(1, 2)) and torch.equal(vt, v.transpose(1, 2))


def test_record_bytes_and_pages_touched():
    assert record_bytes(128, 4) == 4736 and record_bytes(128, 8) == 8832
    assert record_bytes(64, 4) == 2432 and record_bytes(256, 8) == 17536
    assert list(pages_touched(0, 1)) == [0]
    assert list(pages_touched(31, 33)) == [0, 1]
    assert list(pages_touched(32, 32)) == []
    assert list(pages_touched(40, 200)) == [1, 2, 3, 4, 5, 6]


def test_rotation_switch(monkeypatch):
    monkeypatch.delenv("KUSHKASH_ROTATE", raising=False)
    assert rotation_enabled(4) and not rotation_enabled(8)
    assert rotation_enabled(8, True) and not rotation_enabled(4, False)
    monkeypatch.setenv("KUSHKASH_ROTATE", "0")
    assert not rotation_enabled(4)
    monkeypatch.setenv("KUSHKASH_ROTATE", "1")
    assert rotation_enabled(8)
    monkeypatch.setenv("KUSHKASH_ROTATE", "maybe")
    with pytest.raises(ValueError):
        rotation_enabled(4)


def test_fused_write_coverage_check():
    """A one-launch write (Ops.write(fused=True)) needs a job for every page the new rows touch;
    the validation check names the sequence whose list misses one (the last page here, the first
    there) and accepts the complete pages_touched list."""
    from kushkash_amd._ops import _check_covers
    qsl = torch.tensor([0, 40, 40, 100], dtype=torch.int32)     # sequence 1 has no new rows
    sl = torch.tensor([50, 7, 130], dtype=torch.int32)          # 40 rows end at 50; 60 rows end at 130
    full = [(0, p) for p in pages_touched(10, 50)] + [(2, p) for p in pages_touched(70, 130)]

    def check(jobs):
        _check_covers(qsl, sl, torch.tensor([j[0] for j in jobs], dtype=torch.int32),
                      torch.tensor([j[1] for j in jobs], dtype=torch.int32))
    check(full)
    check(full + [(1, 0)])                                       # extra jobs are allowed
    with pytest.raises(ValueError, match="sequence 0 miss touched page"):
        check([j for j in full if j != (0, 1)])                  # the last page of sequence 0
    with pytest.raises(ValueError, match="sequence 2 miss touched page"):
        check([j for j in full if j != (2, 2)])                  # the first page of sequence 2
