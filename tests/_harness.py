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


MANTISSA = {torch.float32: 24, torch.float16: 11, torch.bfloat16: 8}


def half_ulp_of(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Elementwise half an ulp of `dtype` at magnitude |x|: 2^(e - p) for |x| in [2^e, 2^(e+1)) and p
    significant bits (0 at x = 0)."""
    m, e = torch.frexp(x.double().abs())                   # |x| = m 2^e, m in [0.5, 1)
    return torch.where(m > 0, torch.ldexp(torch.ones_like(m), e - 1 - MANTISSA[dtype]), torch.zeros_like(m))


def out_bound(ref: torch.Tensor, dtype: torch.dtype, base: float = 2e-3, roundings: int = 1) -> torch.Tensor:
    """Per-element bound on |out_i - ref_i| for a decode output in `dtype` against an fp32 (or wider)
    reference: `base` (the acceptance bound of the compressed-KV decode: 2e-3 max-abs, fp32
    accumulation) plus, per rounding of the result to `dtype`, half an ulp at |ref_i| + base -- the
    largest magnitude the unrounded result can have, so the ulp is never taken from a smaller binade
    than the one the kernel rounded in. A small output gets the small rounding of its own size, not the
    rounding of the batch's largest value."""
    return base + roundings * half_ulp_of(ref.double().abs() + base, dtype)


def assert_out_close(out: torch.Tensor, ref: torch.Tensor, dtype: torch.dtype, base: float = 2e-3,
                     roundings: int = 1, what: str = "") -> float:
    """Assert |out_i - ref_i| <= out_bound(ref)_i for every element; returns the max-abs error. The
    message names the worst element against its own bound."""
    out, ref = out.detach().double().cpu(), ref.detach().double().cpu()
    assert out.shape == ref.shape, (what, tuple(out.shape), tuple(ref.shape))
    err = (out - ref).abs()
    bound = out_bound(ref, dtype, base, roundings)
    excess = err - bound
    if bool((excess > 0).any()) or bool(torch.isnan(out).any()):
        i = int(torch.nan_to_num(excess, nan=float("inf")).flatten().argmax())
        raise AssertionError(f"{what}: element {i} out {out.flatten()[i].item():.6g} ref {ref.flatten()[i].item():.6g} "
                             f"err {err.flatten()[i].item():.3e} > bound {bound.flatten()[i].item():.3e} "
                             f"({int((excess > 0).sum())} elements over; max-abs {err.max().item():.3e})")
    return err.max().item()
