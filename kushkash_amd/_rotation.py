"""The Walsh-Hadamard rotation of a rotated cache, on the host side: the orthonormal matrix, the
rotation of rows by it (one rounding into the output dtype), the switch that turns it on, and the
canonical butterfly order the kernels evaluate (bit-exact contract).

A rotated cache stores K H and V H and attends with q H, rotating the output back by H (H = H^T =
H^-1); the rotation spreads outlier channels over all dims before the int4 / int8 quantization
(reference: _ops.py:350-377 switch and matrix, :380-395 canonical order, :489-518 rotation).
"""
from __future__ import annotations

import math
import os

import torch

_MATRICES: dict = {}

# fp32 bit patterns of 1 / sqrt(D), the kernels' final scale of the butterflies (quant.mojo:101-110)
FWHT_SCALE_BITS = {64: 0x3E000000, 128: 0x3DB504F3, 256: 0x3D800000}


def rotation_enabled(bits: int, rotate: bool | None = None) -> bool:
    """Whether a cache rotates: `rotate` when given, else the KUSHKASH_ROTATE environment variable --
    "1" on, "0" off, "auto" (the default) on for 4-bit records only; anything else is an error
    (_ops.py:350-359)."""
    if rotate is not None:
        return bool(rotate)
    mode = os.environ.get("KUSHKASH_ROTATE", "auto")
    if mode == "auto":
        return bits == 4
    if mode in ("0", "1"):
        return mode == "1"
    raise ValueError(f"KUSHKASH_ROTATE must be auto, 0 or 1, got {mode}")


def _signs(head_dim: int) -> torch.Tensor:
    """The +-1 Sylvester matrix S_D (S_2n = [[S_n, S_n], [S_n, -S_n]]) as int8 on the CPU."""
    if head_dim < 1 or head_dim & (head_dim - 1):
        raise ValueError(f"Hadamard rotation needs a power-of-2 head_dim, got {head_dim}")
    s = torch.ones(1, 1, dtype=torch.int8)
    step = torch.tensor([[1, 1], [1, -1]], dtype=torch.int8)
    while s.shape[0] < head_dim:
        s = torch.kron(step, s)
    return s


def _matrix(kind: str, head_dim: int, device) -> torch.Tensor:
    key = (kind, head_dim, str(torch.device(device)))
    m = _MATRICES.get(key)
    if m is None:
        s = _signs(head_dim)
        m = (s.double() / math.sqrt(head_dim)).float() if kind == "h" else s.float()
        m = _MATRICES[key] = m.to(device)
    return m


def hadamard(head_dim: int, device) -> torch.Tensor:
    """Orthonormal, symmetric Walsh-Hadamard matrix H [D, D] (H @ H = I) in fp32, Sylvester order,
    cached per (D, device) (_ops.py:362-377)."""
    return _matrix("h", head_dim, device)


def _extent(t: torch.Tensor) -> tuple[int, int]:
    lo = t.data_ptr()
    return lo, lo + t.element_size() * (1 + sum((n - 1) * st for n, st in zip(t.shape, t.stride()) if n > 0))


def _overlap(a: torch.Tensor, b: torch.Tensor) -> bool:
    if a.device != b.device or a.numel() == 0 or b.numel() == 0:
        return False
    (a0, a1), (b0, b1) = _extent(a), _extent(b)
    return a0 < b1 and b0 < a1


def rotate(x: torch.Tensor, h: torch.Tensor | None, dtype: torch.dtype | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """x @ h over the last dim as a contiguous tensor in `dtype` (default x's dtype); h None leaves x as
    it is (cast to `dtype` if given). The product is formed in fp32 against the exact +-1 matrix and
    scaled by fp32 1/sqrt(D), then rounded once into `dtype`, so the result is the orthonormal product
    within one rounding (_ops.py:489-518). H is symmetric with H @ H = I: the same call rotates back.
    out: a contiguous tensor with x's element count in `dtype` that does not overlap x."""
    if h is None:
        y = x if dtype is None else x.to(dtype)
        return y if out is None else out.copy_(y.reshape(out.shape))
    dtype = dtype or x.dtype
    D = h.shape[-1]
    if out is not None:
        if out.numel() != x.numel() or out.dtype != dtype or not out.is_contiguous():
            raise ValueError("rotate(out=): out must be contiguous, in the output dtype, with x's element count")
        if _overlap(out, x):
            raise ValueError("rotate(out=): out overlaps x")
    acc = torch.mm(x.reshape(-1, D).float(), _matrix("s", D, h.device))
    acc.mul_(1.0 / math.sqrt(D))                                  # applied as fp32 1/sqrt(D)
    if out is not None:
        return out.view(-1, D).copy_(acc).view(out.shape)
    return acc.to(dtype).view(x.shape)


def fwht_reference(x: torch.Tensor) -> torch.Tensor:
    """The kernels' canonical Walsh-Hadamard evaluation in torch fp32: butterflies (a, b) -> (a + b,
    a - b) over strides 1, 2, ..., D/2 in that order, then one multiply by the fp32 1/sqrt(D) of
    FWHT_SCALE_BITS (quant.mojo:90-99, _ops.py:383-395)."""
    D = x.shape[-1]
    y = x.float().reshape(-1, D)
    stride = 1
    while stride < D:
        pairs = y.view(y.shape[0], D // (2 * stride), 2, stride)
        y = torch.stack((pairs[:, :, 0] + pairs[:, :, 1], pairs[:, :, 0] - pairs[:, :, 1]), dim=2).reshape(-1, D)
        stride *= 2
    scale = torch.tensor([FWHT_SCALE_BITS[D]], dtype=torch.int32).view(torch.float32).to(y.device)
    return (y * scale).view(x.shape)
