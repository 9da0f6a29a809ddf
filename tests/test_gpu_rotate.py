"""The gfx950 Walsh-Hadamard rotation (needs an MI355X): bit-identical to the oracle's canonical
order (the reference's CPU kernel, restated) for every head_dim and dtype, in place and out of
place, and an involution up to rounding (reference: tests/test_gpu.py:203-218,
tests/test_cpu.py:429-451)."""
import pytest
import torch

import kushkash_amd as kk
from kushkash_amd._ops import fwht_reference, hadamard
from oracle.cpu_ops import OracleOps

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cancelling_rows(D: int, g: torch.Generator) -> torch.Tensor:
    """Rows whose transforms are full of exact zeros, where only the evaluation order fixes the sign
    of each zero: +-0 rows, constants, alternations, +-0 mixed into small integers, repeated blocks,
    halves of opposite sign, subnormal-sized and large values."""
    i = torch.arange(D, dtype=torch.float32)
    rows = [torch.zeros(D), -torch.zeros(D), torch.ones(D), -torch.ones(D), i % 2, (i % 3) - 1,
            torch.where(i % 5 == 0, -0.0, 0.0), torch.where(i < D // 2, 1.0, -1.0), (i % 8 == 0).float() * -1.0,
            torch.full((D,), 1e-38), torch.full((D,), 3e4)]
    for _ in range(40):
        r = torch.randint(-2, 3, (D,), generator=g).float()
        r[torch.rand(D, generator=g) < 0.3] = 0.0
        r[torch.rand(D, generator=g) < 0.3] = -0.0
        rows += [r, torch.randn(D // 8, generator=g).repeat_interleave(8)]
    return torch.stack(rows)


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fwht_gpu_matches_oracle(D, dtype):
    g = torch.Generator().manual_seed(D)
    # 1001 rows: a partial last workgroup; magnitudes 1e-3 .. 1e3 (inputs exact in dtype); then rows
    # whose outputs are mostly zeros, compared bit for bit (the sign of every zero included)
    x = (torch.randn(1001, D, generator=g) * torch.logspace(-3, 3, 1001)[:, None]).to(dtype)
    x = torch.cat([x, _cancelling_rows(D, g).to(dtype)])
    cpu = OracleOps("cpu", D, 4, 1).fwht(x.float().contiguous())
    assert torch.equal(cpu.view(torch.int32), fwht_reference(x.float()).view(torch.int32))
    ops = kk.Ops(torch.device(DEV), D, 4, 1, dtype)
    y = ops.fwht(x.to(DEV)).cpu()
    want = cpu.to(dtype)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    bad = y.view(bits) != want.view(bits)
    assert not bad.any(), f"{bad.sum().item()} of {bad.numel()} values differ from the oracle"
    xc = x.to(DEV)
    assert torch.equal(ops.fwht(xc, out=xc).cpu(), y)                  # in place
    assert ops.fwht(x[:0].to(DEV)).shape == (0, D)
    buf = torch.empty(x.numel() + 1, dtype=dtype, device=DEV)          # rows off 16-byte alignment:
    xo = buf[1:].view(x.shape)                                         # the per-element path
    xo.copy_(x.to(DEV))
    assert torch.equal(ops.fwht(xo).cpu(), y)


@pytest.mark.parametrize("D", [64, 128, 256])
def test_fwht_gpu_is_the_hadamard_rotation(D):
    ops = kk.Ops(torch.device(DEV), D, 4, 1, torch.float32)
    x = torch.randn(3, 5, D, device=DEV)                               # any leading shape
    y = ops.fwht(x)
    dense = x.double().reshape(-1, D) @ hadamard(D, DEV).double()
    assert ((y.reshape(-1, D).double() - dense).norm(dim=1) <= 1e-6 * dense.norm(dim=1)).all()
    back = ops.fwht(y)
    assert ((back - x).norm(dim=-1) <= 1e-6 * x.norm(dim=-1)).all()   # H @ H = I
    with pytest.raises(ValueError):
        ops.fwht(x.double())
    with pytest.raises(ValueError):
        ops.fwht(x.transpose(0, 1))
