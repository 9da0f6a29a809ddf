"""Attention of a chunk of queries over a long key sequence in bounded memory: the keys come in blocks,
each block's (output, log-sum-exp) partial is merged into a running one. Used for prefill chunks over a
quantized history (KushCache.attend_chunk, where the history's blocks are unpacked by the gfx950
unpack kernel; the serving engines' packed prefill, ragged_attention) and as the torch reference of
that path (history_attention, where they are dequantized by torch). Reference semantics:
kushkash/_ops.py:254-285 (attention with log-sum-exp, merge), :309-339 (history attention).

Two ways to attend a block: torch products in fp32 (the reference path, and any input the fused
kernel does not take), or, where the caller asks for it (`fused`), torch's flash-attention kernel on
the GPU for bf16 / fp16 inputs, which returns the log-sum-exp the merges need, takes the GQA head
groups and aligns a causal block's queries with its last keys -- what the reference uses where its
platform has it (_ops.py:254-276, vllm/backend.py:837-880). KUSHKASH_ATTN=fp32 keeps the products.

Memory: with the products, a block's score matrix [B, Hk, G*T, n] fp32 (and its exponentials) and its
K / V in fp32 are what a block costs; the block length n is chosen so that they stay within
`block_bytes`, whatever the history's length and the chunk's size (the chunk's own keys are blocked
the same way). The fused kernel keeps no score matrix: only K / V bound its blocks.
"""
from __future__ import annotations

import os
from functools import lru_cache

import torch

from ._records import PAGE, as_records, dequant_records


@lru_cache(None)
def _flash_takes(dtype: torch.dtype, head_dim: int, device: torch.device) -> bool:
    """Whether torch's flash-attention kernel runs for this dtype and head size on this device: one call
    on a single query and key, once per process and shape."""
    x = torch.zeros(1, 1, 1, head_dim, dtype=dtype, device=device)
    try:
        torch.ops.aten._flash_attention_forward(x, x, x, None, None, 1, 1, 0.0, False, False, scale=1.0)
        return True
    except RuntimeError:
        return False


def fused_ok(q: torch.Tensor) -> bool:
    """Whether torch's flash-attention kernel takes q: bf16 / fp16 on the GPU at a head size it runs,
    unless KUSHKASH_ATTN=fp32. Block sizes follow this answer, so a refused shape never gets blocks
    sized for the fused kernel."""
    return (q.is_cuda and q.dtype in (torch.bfloat16, torch.float16) and os.environ.get("KUSHKASH_ATTN") != "fp32"
            and _flash_takes(q.dtype, q.shape[-1], q.device))


def _flash(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, scale: float):
    """attn_lse by torch's flash-attention kernel, or None where it refuses the shape. Without a mask
    the q heads of a kv head are folded into its query rows (one kernel head per kv head); causal
    blocks pass the head groups to the kernel, which aligns the queries with the last T keys."""
    B, Hq, T, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    g = Hq // Hk
    kt, vt = k.transpose(1, 2).contiguous(), v.transpose(1, 2).contiguous()           # [B, N, Hk, D]
    try:
        if causal:
            o, lse = torch.ops.aten._flash_attention_forward(
                q.transpose(1, 2).contiguous(), kt, vt, None, None, T, N, 0.0, True, False, scale=scale)[:2]
            return o.transpose(1, 2).float(), lse[..., :T].float()
        qf = q.reshape(B, Hk, g * T, D).transpose(1, 2).contiguous()                    # [B, gT, Hk, D]
        o, lse = torch.ops.aten._flash_attention_forward(qf, kt, vt, None, None, g * T, N, 0.0, False, False,
                                                         scale=scale)[:2]
        return (o.transpose(1, 2).reshape(B, Hq, T, D).float(),
                lse[..., :g * T].reshape(B, Hq, T).float())
    except RuntimeError:
        return None


def attn_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, scale: float,
             key_offset: int | None = None, fused: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """(out fp32 [B, Hq, T, D], log-sum-exp fp32 [B, Hq, T]) of q [B, Hq, T, D] over k, v [B, Hk, N, D]
    (GQA: q head i reads kv head i // (Hq / Hk)). The q heads of a kv head are folded into its query
    rows, so K and V are never expanded. causal: query t sees keys j <= key_offset + t (default
    N - T: the queries are the last T of the keys); a query that sees no key gets out 0 and lse -inf
    (_ops.py:254-276). fused: torch's flash-attention kernel where it takes the input (no mask, or
    the default causal alignment with N >= T), else the fp32 products."""
    B, Hq, T, D = q.shape
    Hk, N = k.shape[1], k.shape[2]
    if fused and fused_ok(q) and N > 0 and (not causal or ((key_offset is None or key_offset == N - T) and N >= T)):
        r = _flash(q, k, v, causal, scale)
        if r is not None:
            return r
        n = keys_per_block(q, Hk, 2 * B * Hk * D * 4, 1 << 28, 1)     # refused: products, scores bounded
        if not causal and n < N:
            acc = None
            for j0 in range(0, N, n):
                acc = merge(acc, attn_lse(q, k[:, :, j0:j0 + n], v[:, :, j0:j0 + n], False, scale))
            return acc
    g = Hq // Hk
    qf = q.reshape(B, Hk, g * T, D).float()
    s = torch.matmul(qf, k.float().transpose(-1, -2).contiguous()).mul_(scale)      # [B, Hk, gT, N]
    if causal:
        off = N - T if key_offset is None else key_offset
        t = torch.arange(T, device=q.device).repeat(g)                               # row -> query index
        hidden = torch.arange(N, device=q.device)[None, :] > (t[:, None] + off)
        s.masked_fill_(hidden, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)                                                  # [B, Hk, gT]
    base = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
    p = torch.exp(s.sub_(base.unsqueeze(-1)))                                         # rows with no key: 0
    out = torch.matmul(p, v.float())
    return out.view(B, Hq, T, D), lse.view(B, Hq, T)


def merge(acc, part):
    """Combine (out, lse) partials of the same queries over disjoint key sets: out = the partials
    weighted by their share of the total exp-sum, lse = log of the total (_ops.py:279-285). acc None
    -> part. A side over no keys (lse -inf) gets weight 0."""
    if acc is None:
        return part
    (o1, l1), (o2, l2) = acc, part
    w1 = torch.sigmoid(torch.nan_to_num(l1 - l2, nan=0.0))           # e^l1 / (e^l1 + e^l2)
    return torch.lerp(o2, o1, w1.unsqueeze(-1)), torch.logaddexp(l1, l2)


def keys_per_block(q: torch.Tensor, n_kv_heads: int, kv_bytes_per_key: int, block_bytes: int, quantum: int,
                   scores: bool = True) -> int:
    """Keys per block so that one block's scores and exponentials (fp32, 2 x 4 bytes per query row and
    key; none with scores=False, the fused kernel) and its K / V (kv_bytes_per_key per key, all kv heads
    and batch) fit in block_bytes; a multiple of `quantum`, at least one quantum."""
    B, Hq, T, _ = q.shape
    per_key = (8 * B * Hq * T if scores else 0) + kv_bytes_per_key
    return max(quantum, (block_bytes // per_key) // quantum * quantum)


def self_attention_blocks(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, scale: float,
                          block_bytes: int, acc=None, fused: bool = False):
    """Merge into acc the causal attention of the T queries of q over the chunk's own T keys (query t
    sees chunk keys 0..t), the keys in blocks that keep the scores within block_bytes (fused: one
    block, the flash-attention kernel, where it takes q)."""
    T, D = q.shape[2], q.shape[3]
    B, Hk = k_new.shape[0], k_new.shape[1]
    if fused and fused_ok(q) and T > 0:
        r = _flash(q, k_new, v_new, True, scale)
        if r is not None:
            return merge(acc, r)
    n = keys_per_block(q, Hk, 2 * B * Hk * D * 4, block_bytes, 1)
    for j0 in range(0, T, n):
        j1 = min(T, j0 + n)
        acc = merge(acc, attn_lse(q, k_new[:, :, j0:j1], v_new[:, :, j0:j1], True, scale, key_offset=-j0))
    return acc


def ragged_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_start: list, k_start: list, scale: float,
                     block_bytes: int = 1 << 28, varlen: tuple | None = None) -> torch.Tensor:
    """Causal attention of ragged rows packed end to end: row i's queries q[q_start[i]:q_start[i+1]]
    ([rows, Hq, D]) over its keys k, v[k_start[i]:k_start[i+1]] ([rows, Hk, D]), the queries being the
    last T of the row's N keys (query t sees keys j <= N - T + t: the serving engines' prefill
    convention). varlen = (cu_q, cu_k, max_q, max_k), the offsets as int32 device tensors: every row in
    one launch of torch's flash-attention kernel (varlen form) where it takes q and no row is empty;
    otherwise fp32 products per row, keys in blocks that keep each block's scores within block_bytes.
    Returns q's shape and dtype."""
    if (varlen is not None and fused_ok(q)
            and all(b > a for a, b in zip(q_start[:-1], q_start[1:]))):
        cu_q, cu_k, max_q, max_k = varlen
        try:
            return torch.ops.aten._flash_attention_forward(q, k, v, cu_q, cu_k, max_q, max_k, 0.0, True, False,
                                                           scale=scale)[0]
        except RuntimeError:
            pass
    out = q.new_empty(q.shape)
    Hk, D = k.shape[1], k.shape[2]
    for i in range(len(q_start) - 1):
        a, b, c, d = q_start[i], q_start[i + 1], k_start[i], k_start[i + 1]
        if b <= a:
            continue
        T, N = b - a, d - c
        qi = q[a:b].transpose(0, 1).unsqueeze(0)                               # [1, Hq, T, D]
        ki = k[c:d].transpose(0, 1).unsqueeze(0)                               # [1, Hk, N, D]
        vi = v[c:d].transpose(0, 1).unsqueeze(0)
        n = keys_per_block(qi, Hk, 2 * Hk * D * 4, block_bytes, 1)
        acc = None
        for j0 in range(0, N, n):
            j1 = min(N, j0 + n)
            acc = merge(acc, attn_lse(qi, ki[:, :, j0:j1], vi[:, :, j0:j1], True, scale, key_offset=N - T - j0))
        out[a:b] = acc[0][0].transpose(0, 1).to(q.dtype)
    return out


def history_attention(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, records: torch.Tensor,
                      block_ids: torch.Tensor, n_hist: int, tail_k: torch.Tensor, head_dim: int, bits: int,
                      scale: float, block_bytes: int = 1 << 28) -> torch.Tensor:
    """Attention of T new queries over n_hist cached tokens plus the T new tokens themselves (causal),
    the torch reference path: history pages dequantized by torch a block at a time (the partial page
    with its exact K from tail_k [B, Hk, 32, D]), every partial merged by log-sum-exp, memory bounded
    by block_bytes (_ops.py:309-339). q [B, Hq, T, D]; k_new, v_new [B, Hk, T, D]; returns [B, Hq, T, D]
    in q's dtype."""
    B, Hk, D = q.shape[0], k_new.shape[1], head_dim
    recs = as_records(records)
    acc = None
    full = n_hist // PAGE
    if n_hist:
        step = keys_per_block(q, Hk, 2 * B * Hk * D * (4 + q.element_size()), block_bytes, PAGE) // PAGE
        for p0 in range(0, full, step):
            p1 = min(full, p0 + step)
            k, v = dequant_records(recs[block_ids[:, p0:p1].long()], D, bits, q.dtype, token_major=True)
            # [B, pages, 32, Hk, D] -> [B, Hk, pages * 32, D]
            k = k.flatten(1, 2).transpose(1, 2)
            v = v.flatten(1, 2).transpose(1, 2)
            acc = merge(acc, attn_lse(q, k, v, False, scale))
        r = n_hist - full * PAGE
        if r:
            v = dequant_records(recs[block_ids[:, full].long()], D, bits, q.dtype)[1]       # [B, Hk, 32, D]
            acc = merge(acc, attn_lse(q, tail_k[:, :, :r].to(q.dtype), v[:, :, :r], False, scale))
    acc = self_attention_blocks(q, k_new.to(q.dtype), v_new.to(q.dtype), scale, block_bytes, acc)
    return acc[0].to(q.dtype)


def unpacked_history_attention(ops, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, cache: torch.Tensor,
                               block_table: torch.Tensor, n_hist: int, tail_k: torch.Tensor, tail_idx: torch.Tensor,
                               scale: float, rot: bool, block_bytes: int = 1 << 28) -> torch.Tensor:
    """history_attention on the GPU kernels: each block of history pages (all B sequences) is unpacked
    into K / V rows by one launch of the unpack kernel (Ops.unpack: fma(code, scale, bias) in fp32, one
    rounding to the cache dtype; rot rotates a rotated cache's rows back, so the attention runs on the
    unrotated q and chunk), the partial page's K from the tail slots tail_idx. Shapes as
    history_attention; returns [B, Hq, T, D] in q's dtype."""
    B, Hq, T, D = q.shape
    Hk = k_new.shape[1]
    dev, dt = q.device, ops.dtype
    acc = None
    full = n_hist // PAGE
    r = n_hist - full * PAGE
    if n_hist:
        fused = fused_ok(q)
        step = keys_per_block(q, Hk, 2 * B * Hk * D * (4 + torch.finfo(dt).bits // 8), block_bytes, PAGE,
                              scores=not fused) // PAGE
        none = torch.zeros(0, dtype=torch.int32, device=dev)
        empty = torch.zeros(0, Hk, D, dtype=dt, device=dev)
        p0 = 0
        while p0 < full or (p0 == full and r):
            p1 = min(full, p0 + step)
            tail = r > 0 and p1 == full                      # the partial page rides with the last block
            npg = p1 - p0 + (1 if tail else 0)
            rows = npg * PAGE
            kp = torch.empty(B * rows, Hk, D, dtype=dt, device=dev)
            vp = torch.empty_like(kp)
            seq0 = torch.arange(B, device=dev, dtype=torch.int32) * rows
            blk = block_table[:, p0:p1].contiguous().view(-1)
            dst = (seq0[:, None] + torch.arange(p1 - p0, device=dev, dtype=torch.int32)[None, :] * PAGE).view(-1)
            if tail:
                tail_blk = block_table[:, full].contiguous()
                info = torch.stack([seq0 + (p1 - p0) * PAGE, torch.full_like(seq0, r), tail_idx[:B].to(torch.int32)],
                                   dim=1).view(-1)
            else:
                tail_blk = info = none
            ops.unpack(cache, blk, dst.contiguous(), tail_blk, info.contiguous(), tail_k, empty, empty, none, kp, vp,
                       rot)
            n = (p1 - p0) * PAGE + (r if tail else 0)
            k = kp.view(B, rows, Hk, D)[:, :n].transpose(1, 2)
            v = vp.view(B, rows, Hk, D)[:, :n].transpose(1, 2)
            acc = merge(acc, attn_lse(q, k, v, False, scale, fused=True))
            p0 = p1 + (1 if tail else 0)
    acc = self_attention_blocks(q, k_new.to(q.dtype), v_new.to(q.dtype), scale, block_bytes, acc, fused=True)
    return acc[0].to(q.dtype)
