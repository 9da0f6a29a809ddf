"""Shared test helpers: the oracle-backed CPU cache, reference restatements from the reference's
own tests, and tolerance helpers."""
from __future__ import annotations

import contextlib
import math

import torch

import kushkash_amd
from kushkash_amd import cache as cache_mod
from kushkash_amd._ops import PAGE
from oracle.cpu_ops import OracleOps


@contextlib.contextmanager
def oracle_backend():
    """KushCache(device="cpu") built inside this block runs on the CPU oracle (test-side only)."""
    real = cache_mod.Ops
    cache_mod.Ops = OracleOps
    try:
        yield
    finally:
        cache_mod.Ops = real


def oracle_cache(*args, **kw) -> kushkash_amd.KushCache:
    kw = dict(kw, device="cpu", dtype=torch.float32)
    with oracle_backend():
        return kushkash_amd.KushCache(*args, **kw)


def ref_quantize(x: torch.Tensor, bits: int, dim: int):
    """The reference test's torch restatement of the format (tests/test_cpu.py:16-24): codes,
    fp16-rounded scale and bias over `dim`."""
    levels, half = 2 ** bits - 1, 2 ** (bits - 1)
    mn, mx = x.amin(dim, keepdim=True), x.amax(dim, keepdim=True)
    s = ((mx - mn) / levels).half().float()
    b = (mn + s * half).half().float()
    inv = torch.where(s > 0, 1.0 / s, torch.zeros_like(s))
    c = torch.round((x - b) * inv).clamp(-half, half - 1).to(torch.int8)
    return c, s, b


def ref_dequant(x: torch.Tensor, bits: int, dim: int) -> torch.Tensor:
    """Quantize -> dequantize of groups along `dim` (tests/test_ragged.py:17-24)."""
    c, s, b = ref_quantize(x, bits, dim)
    return c.float() * s + b


def split_record(rec: torch.Tensor, D: int, bits: int):
    """Record bytes [..., RB] -> (k codes [..., 32, D], ks, kb [..., D], v codes, vs, vb [..., 32])
    (tests/test_cpu.py:27-37)."""
    dc = D if bits == 8 else D // 2

    def unpack(c):
        return torch.cat([(c << 4) >> 4, c >> 4], -1) if bits == 4 else c

    kq = unpack(rec[..., :PAGE * dc].view(torch.int8).unflatten(-1, (PAGE, dc)))
    vq = unpack(rec[..., PAGE * dc:2 * PAGE * dc].view(torch.int8).unflatten(-1, (PAGE, dc)))
    meta = rec[..., 2 * PAGE * dc:].contiguous().view(torch.float16).float()
    return kq, meta[..., :D], meta[..., D:2 * D], vq, meta[..., 2 * D:2 * D + PAGE], meta[..., 2 * D + PAGE:]


def half_ulp(x: float, dtype: torch.dtype) -> float:
    """Half an ulp of `dtype` at magnitude |x| (the largest rounding error of a value of that size):
    2^(e - p) for |x| in [2^e, 2^(e+1)) and p significant bits (fp32 24, fp16 11, bf16 8)."""
    p = {torch.float32: 24, torch.float16: 11, torch.bfloat16: 8}[dtype]
    x = abs(float(x))
    if x == 0.0:
        return 0.0
    e = math.frexp(x)[1] - 1                       # x = m 2^(e+1), m in [0.5, 1)
    return math.ldexp(1.0, e - p)


def out_tol(ref: torch.Tensor, dtype: torch.dtype, base: float = 2e-3) -> float:
    """Max-abs tolerance of a decode output in `dtype` against an fp32 reference: `base` plus half an
    ulp of the output dtype at the largest |ref| (the rounding of the output itself; no element of
    smaller magnitude rounds further)."""
    return base + half_ulp(float(ref.abs().max()), dtype)
