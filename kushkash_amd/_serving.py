"""Diagnostics and fallback switches of the serving integrations (vLLM CUSTOM backend, SGLang
backend), with the reference's names and meanings (kushkash/vllm/backend.py:66-67, :80-85, :219-226,
:646-658, :738-790; kushkash/sglang/backend.py:45-48). Each is read from the environment when it is
used, so a serving process (or a test) can set it before the step that should see it.

    KUSHKASH_SYNC=1          serialize host and device after every attention call (outside graph capture)
    KUSHKASH_CHECK=<path>    layer 0 of every step (the first 400 calls): the output checked against torch
                             attention over the cache's own dequantized records, relative errors appended
                             to <path>, one line per call
    KUSHKASH_MEM_STATS=N     every N packed-prefill steps, layer 0 prints the torch allocator's counters
    KUSHKASH_PROFILE_STEP=0  vLLM's memory profiling reserves no prefill temporaries (escape hatch)
    KUSHKASH_UNPACK=torch    packed prefill builds its keys / values with torch (gather, dequantize,
                             rotate back, scatter) instead of the unpack kernel, for A/B comparisons;
                             default: kernel (the reference's name for its kernel path, mojo, is accepted)
"""
from __future__ import annotations

import os
import sys

import torch

from ._records import PAGE, as_records, cached_kv, dequant_records
from ._rotation import fwht_reference

CHECK_CALLS = 400                 # KUSHKASH_CHECK stops logging after this many calls (per process)
_check_calls = [0]


def sync_enabled() -> bool:
    return os.environ.get("KUSHKASH_SYNC", "0") == "1"


def check_path() -> str:
    return os.environ.get("KUSHKASH_CHECK", "")


def mem_stats_every() -> int:
    value = os.environ.get("KUSHKASH_MEM_STATS", "0").strip() or "0"
    n = int(value)
    if n < 0:
        raise ValueError("KUSHKASH_MEM_STATS must be >= 0")
    return n


def profile_step_enabled() -> bool:
    return os.environ.get("KUSHKASH_PROFILE_STEP", "1") != "0"


def unpack_mode() -> str:
    """kernel (default; `mojo`, the reference's name for its kernel path, means the same) or torch."""
    mode = os.environ.get("KUSHKASH_UNPACK", "kernel").strip().lower()
    if mode in ("kernel", "mojo", "hip"):
        return "kernel"
    if mode != "torch":
        raise ValueError("KUSHKASH_UNPACK must be kernel (or mojo) or torch")
    return mode


def capturing(t: torch.Tensor) -> bool:
    return t.is_cuda and torch.cuda.is_current_stream_capturing()


def maybe_sync(t: torch.Tensor) -> None:
    """KUSHKASH_SYNC=1: wait for the device after an attention call (never inside a graph capture)."""
    if sync_enabled() and t.is_cuda and not capturing(t):
        torch.cuda.synchronize(t.device)


class MemStats:
    """KUSHKASH_MEM_STATS=N: counts packed-prefill steps (one owner per engine calls tick once a step)
    and every N-th prints the allocator's retry / OOM counters and current sizes to stderr."""

    def __init__(self):
        self.steps = 0

    def tick(self, device: torch.device) -> str | None:
        every = mem_stats_every()
        if not every or device.type != "cuda" or torch.cuda.is_current_stream_capturing():
            return None
        self.steps += 1
        if self.steps % every:
            return None
        st = torch.cuda.memory_stats(device)
        line = (f"kushkash mem: packed steps {self.steps}, alloc retries {st.get('num_alloc_retries', 0)}, "
                f"OOMs {st.get('num_ooms', 0)}, allocated {st.get('allocated_bytes.all.current', 0) >> 20} MiB, "
                f"reserved {st.get('reserved_bytes.all.current', 0) >> 20} MiB, inactive split "
                f"{st.get('inactive_split_bytes.all.current', 0) >> 20} MiB")
        print(line, file=sys.stderr, flush=True)
        return line


def torch_unpack(cache: torch.Tensor, page_blk: torch.Tensor, page_dst: torch.Tensor, tail_blk: torch.Tensor,
                 tail_info: torch.Tensor, tail_k: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                 new_dst: torch.Tensor, kp: torch.Tensor, vp: torch.Tensor, head_dim: int, bits: int, rot: bool,
                 pages_per_slice: int = 256) -> None:
    """KUSHKASH_UNPACK=torch: what Ops.unpack writes, built with torch (the reference's torch packed
    path, kushkash/vllm/backend.py:858-878): full history pages (block page_blk[i] -> rows page_dst[i]
    + 0..31) dequantized a slice of pages at a time; partial pages (block tail_blk[i], tail_info[i] =
    (first row, tokens, tail slot)) with K from the tail and V from the record; the new rows copied.
    Dequantization in fp32 (code * scale exact, + bias rounded once), rotated back by the canonical
    Walsh-Hadamard order in fp32 when rot, then one rounding to kp's dtype: the unpack kernel's
    arithmetic, so both give the same bits."""
    recs = as_records(cache)
    H, D, dtype = kp.shape[1], head_dim, kp.dtype
    ar = torch.arange(PAGE, device=kp.device)

    def finish(x):                                   # fp32 rows -> (rotated back) -> dtype
        return (fwht_reference(x) if rot else x).to(dtype)

    n_pages = page_blk.numel()
    for p0 in range(0, n_pages, pages_per_slice):
        p1 = min(n_pages, p0 + pages_per_slice)
        k, v = dequant_records(recs[page_blk[p0:p1].long(), :H], D, bits, torch.float32, token_major=True)
        rows = (page_dst[p0:p1].long()[:, None] + ar).reshape(-1)            # [n * 32]
        kp.index_copy_(0, rows, finish(k).reshape(-1, H, D))
        vp.index_copy_(0, rows, finish(v).reshape(-1, H, D))
    info = tail_info.view(-1, 3).long().cpu().tolist() if tail_blk.numel() else []
    blocks = tail_blk.long().cpu().tolist()
    for i, (first, n, slot) in enumerate(info):
        if n <= 0:
            continue
        _, v = dequant_records(recs[blocks[i]][:H], D, bits, torch.float32, token_major=True)
        k = tail_k[slot, :H, :n].float().transpose(0, 1)                     # [n, H, D], exact (rotated) K
        kp[first:first + n] = finish(k)
        vp[first:first + n] = finish(v[:n])
    if new_dst.numel():
        kp.index_copy_(0, new_dst.long(), k_new[:new_dst.numel()])
        vp.index_copy_(0, new_dst.long(), v_new[:new_dst.numel()])


def reference_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """fp32 attention of q [T, Hq, D] over k, v [Hk, n, D] (q head i reads kv head i // (Hq / Hk));
    the T queries are the last T positions of the n keys (causal within them)."""
    T, Hq, _ = q.shape
    Hk, n = k.shape[0], k.shape[1]
    g = Hq // Hk
    mask = torch.ones(T, n, dtype=torch.bool, device=q.device).tril(diagonal=n - T)
    # explicit fp32 products (no fused-attention backend is chosen for this check)
    kk = k.float().repeat_interleave(g, 0)                                   # [Hq, n, D]
    vv = v.float().repeat_interleave(g, 0)
    s = torch.matmul(q.float().transpose(0, 1).contiguous(), kk.transpose(1, 2).contiguous()) * scale
    p = torch.softmax(s.masked_fill(~mask, float("-inf")), dim=-1)
    return torch.matmul(p, vv).transpose(0, 1)


class Checker:
    """KUSHKASH_CHECK=<path>: the attention outputs of one call checked against torch attention over
    the cache's own records (dequantized in fp32, the partial page's K exact from its tail; rotated
    back when the cache is rotated), one line per call appended to <path>: per request 'd' (decode) or
    'p' (prefill), its length, query rows and tail slot, and the relative error |out - ref| / |ref|.
    Prefill references are taken before the step's write (the cache then holds the history only, the
    new rows come from the call's own k / v); decode references after the call (its token appended)."""

    def __init__(self, head_dim: int, bits: int, scale: float, rot: bool):
        self.D, self.bits, self.scale, self.rot = head_dim, bits, scale, rot

    @staticmethod
    def wanted(q: torch.Tensor, first_layer: bool) -> bool:
        return bool(check_path()) and first_layer and not capturing(q) and _check_calls[0] < CHECK_CALLS

    def _history(self, cache, block_table, tail, slot, n):
        """Cached K, V [Hk, n, D] of one request in the model's space, fp32."""
        if n == 0:
            H = tail.shape[1]
            z = torch.zeros(H, 0, self.D, device=tail.device)
            return z, z
        k, v = cached_kv(cache, block_table[None], n, tail[slot:slot + 1], self.D, self.bits, torch.float32)
        if self.rot:
            k, v = fwht_reference(k), fwht_reference(v)
        return k[0], v[0]

    def prefill_refs(self, q, k_new, v_new, cache, block_table, tail, slots, q_start, history, rows):
        """References of prefill requests `rows` (indices into the step's requests), before the write."""
        refs = {}
        for r in rows:
            a, b = q_start[r], q_start[r + 1]
            K, V = self._history(cache, block_table[r], tail, int(slots[r]), history[r])
            K = torch.cat([K, k_new[a:b].float().transpose(0, 1)], 1)
            V = torch.cat([V, v_new[a:b].float().transpose(0, 1)], 1)
            refs[r] = reference_attention(q[a:b], K, V, self.scale)
        return refs

    def log(self, out, q, cache, block_table, tail, slots, q_start, seq_lens, n_decodes, prefill_refs) -> str:
        """Checks every request of the call and appends the line to the log; returns it."""
        _check_calls[0] += 1
        errs = []
        for r in range(len(q_start) - 1):
            a, b = q_start[r], q_start[r + 1]
            if b <= a:
                continue
            if r < n_decodes:
                K, V = self._history(cache, block_table[r], tail, int(slots[r]), seq_lens[r])
                ref = reference_attention(q[a:b], K, V, self.scale)
            else:
                ref = prefill_refs[r]
            e = float((out[a:b].float() - ref).norm() / ref.norm().clamp_min(1e-6))
            kind = "d" if r < n_decodes else "p"
            errs.append(f"{kind}{r}:len{seq_lens[r]}/q{b - a}/slot{int(slots[r])}:{e:.1e}")
        line = (f"call {_check_calls[0]} rows={len(q_start) - 1} dec={n_decodes} tokens={q_start[-1]} | "
                + " ".join(errs))
        with open(check_path(), "a") as f:
            f.write(line + "\n")
        return line


def max_check_error(line: str) -> float:
    """The largest relative error of a KUSHKASH_CHECK line (for tests and log readers)."""
    vals = [float(x.rsplit(":", 1)[1]) for x in line.split(" | ", 1)[1].split()] if " | " in line else []
    return max(vals) if vals else 0.0
