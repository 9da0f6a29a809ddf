"""Torch view of page records, for references and tests: a record's codes and fp16 parameters turned
back into K / V values, and the cached K / V of a batch laid out token by token.

The record format is the reference's (quant.mojo:53-87): per (page, kv head)
    [K codes 32 x DC | V codes 32 x DC | K scale D | K bias D | V scale 32 | V bias 32]
with DC = D (int8) or D / 2 (int4: byte j holds dim j in its low nibble and dim j + D/2 in its high
nibble, both two's complement), the parameters fp16. A value is code * scale + bias
(_ops.py:217-251 dequant_records, :295-306 cached_kv). Here the product and the sum are formed in
fp32 -- the product of a code and an fp16 scale is exact there -- and rounded once to the output
dtype, as the unpack kernel rounds them.
"""
from __future__ import annotations

import torch

PAGE = 32


def _code_bytes(head_dim: int, bits: int) -> int:
    return head_dim if bits == 8 else head_dim // 2


def _nibbles(b: torch.Tensor) -> torch.Tensor:
    """int4 code bytes [..., D/2] -> signed codes [..., D]: low nibbles are dims 0..D/2-1, high nibbles
    the rest; ((x & 15) ^ 8) - 8 sign-extends a nibble, an arithmetic shift the high one."""
    return torch.cat([((b & 15) ^ 8) - 8, b >> 4], dim=-1)


def record_fields(rec: torch.Tensor, head_dim: int, bits: int):
    """Records [..., RB] (uint8) -> (K codes, V codes [..., 32, D] int8, K scale, K bias [..., D], V
    scale, V bias [..., 32]) with the parameters as fp32."""
    dc = _code_bytes(head_dim, bits)
    body = 2 * PAGE * dc
    codes = rec[..., :body].view(torch.int8).unflatten(-1, (2, PAGE, dc))
    if bits == 4:
        codes = _nibbles(codes)
    par = rec[..., body:body + 2 * (2 * head_dim + 2 * PAGE)].contiguous().view(torch.float16).float()
    ks, kb, vs, vb = par.split([head_dim, head_dim, PAGE, PAGE], dim=-1)
    return codes[..., 0, :, :], codes[..., 1, :, :], ks, kb, vs, vb


def dequant_records(rec: torch.Tensor, head_dim: int, bits: int, dtype: torch.dtype, token_major: bool = False,
                    out: tuple[torch.Tensor | None, torch.Tensor | None] | None = None
                    ) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """Records [..., RB] -> K, V [..., 32, D] in `dtype` (contiguous). token_major: records
    [..., H, RB] -> [..., 32, H, D]. out: (k, v) contiguous tensors of that shape and dtype to fill; a
    None entry skips that half (and returns None for it). Reference: _ops.py:217-251."""
    kc, vc, ks, kb, vs, vb = record_fields(rec, head_dim, bits)
    halves = ((kc, ks.unsqueeze(-2), kb.unsqueeze(-2)), (vc, vs.unsqueeze(-1), vb.unsqueeze(-1)))
    dst = out if out is not None else (None, None)
    result = []
    for i, (c, s, b) in enumerate(halves):
        if out is not None and dst[i] is None:
            result.append(None)
            continue
        x = torch.addcmul(b, c.float(), s)                      # fp32: c * s exact, one rounding for + b
        if token_major:
            x = x.transpose(-3, -2)
        if dst[i] is None:
            result.append(x.to(dtype).contiguous())
        else:
            if dst[i].shape != x.shape or dst[i].dtype != dtype or not dst[i].is_contiguous():
                raise ValueError(f"dequant_records(out=): need a contiguous {dtype} {tuple(x.shape)} tensor, got "
                                 f"{dst[i].dtype} {tuple(dst[i].shape)}")
            result.append(dst[i].copy_(x))
    return result[0], result[1]


def as_records(cache: torch.Tensor) -> torch.Tensor:
    """A cache tensor whose dim 0 is the block and dim 1 the kv head, with each record's bytes
    contiguous ([blocks, H, RB] uint8, or a vLLM-style [blocks, H, 32, C] view of another dtype), as
    uint8 [blocks, H, RB] (_ops.py:288-292)."""
    c = cache.view(torch.uint8) if cache.dtype != torch.uint8 else cache
    return c if c.dim() == 3 else c.flatten(2)


def cached_kv(records: torch.Tensor, block_ids: torch.Tensor, n: int, tail_k: torch.Tensor, head_dim: int, bits: int,
              dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """The first n cached tokens of each of B sequences as K, V [B, Hk, n, D] in `dtype`: full pages
    from their records (block ids block_ids[b, :pages]); on a partial last page, K from the exact tail
    tail_k [B, Hk, 32, D] and V from the page's record (_ops.py:295-306)."""
    recs = as_records(records)
    B, Hk = block_ids.shape[0], tail_k.shape[1]
    pages = -(-n // PAGE)
    full = n // PAGE
    k, v = dequant_records(recs[block_ids[:, :pages].long()], head_dim, bits, dtype, token_major=False)
    # [B, pages, Hk, 32, D] -> [B, Hk, pages * 32, D]
    k = k.permute(0, 2, 1, 3, 4).reshape(B, Hk, pages * PAGE, head_dim)
    v = v.permute(0, 2, 1, 3, 4).reshape(B, Hk, pages * PAGE, head_dim)
    if n > full * PAGE:
        k[:, :, full * PAGE:] = tail_k.to(dtype)                  # the tail's exact K (its later rows are cut)
    return k[:, :, :n].contiguous(), v[:, :, :n].contiguous()
