"""Prefill (extend) steps over page records, shared by the serving integrations (SGLang, vLLM): a ragged
batch of requests, request r holding history[r] cached tokens (its last page possibly unfinished, with
that page's exact K in the request's tail slot) and adding new_tokens[r] tokens this step, whose
queries attend to the whole history and causally to each other.
Reference semantics: the packed prefill of kushkash/sglang/backend.py:53-105, :256-291, :367-398 and
kushkash/vllm/backend.py:385-475, :807-880.

Host side, once per step (``ExtendPlan``): the write jobs (one per (request, logical page) the new
tokens touch), and the attention groups: consecutive requests whose K + V, history and new tokens
together, fit a byte budget are packed end to end; a request over the budget alone (and every request
in loop mode) takes its history in blocks of pages. All index arrays go to the device in one copy.

Device side, per layer (``ExtendPlan.attend``, before the step's write): per packed group one launch of
the unpack kernel builds every request's keys [history pages | partial page (K from the tail, V from
its record) | new tokens] in the model dtype -- rotated back when the cache is rotated, so attention
runs on the model's own q, k, v -- and a causal ragged attention runs over them (a group with no
history skips the unpack and attends over the new rows directly); a blocked request unpacks its
history a block of pages at a time and merges the blocks by log-sum-exp. Then ``ExtendPlan.write``
quantizes the new tokens with one write launch.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

import numpy as np
import torch

from ._attention import ragged_attention, unpacked_history_attention
from ._ops import PAGE, pages_touched
from ._serving import torch_unpack, unpack_mode


def record_bits() -> int:
    """Record bits of a serving cache: KUSHKASH_BITS, 4 (default) or 8."""
    value = os.environ.get("KUSHKASH_BITS", "4")
    if value not in ("4", "8"):
        raise ValueError(f"KUSHKASH_BITS must be 4 or 8, got {value}")
    return int(value)


def pack_budget() -> int:
    """Bytes of K + V one packed group may hold: KUSHKASH_PACK_MB MiB (auto or unset: 512)."""
    value = os.environ.get("KUSHKASH_PACK_MB", "auto").strip().lower()
    mb = 512 if value in ("", "auto") else int(value)
    if mb < 0:
        raise ValueError("KUSHKASH_PACK_MB must be >= 0 or auto")
    return mb << 20


def prefill_mode() -> str:
    """KUSHKASH_PREFILL: packed (default: requests packed into groups) or loop (each request on its own)."""
    mode = os.environ.get("KUSHKASH_PREFILL", "packed")
    if mode not in ("packed", "loop"):
        raise ValueError(f"KUSHKASH_PREFILL must be packed or loop, got {mode}")
    return mode


@dataclass
class PackPlan:
    """Where each key of a packed buffer comes from. Request r's keys occupy packed rows
    [key_start[r], key_start[r + 1]): its full history pages, then the tokens of its partial page (K
    from the tail, V from the page's record), then its new tokens. numpy int64 arrays."""
    key_start: np.ndarray    # [R + 1]
    page_req: np.ndarray     # per full history page: request,
    page_index: np.ndarray   #   logical page,
    page_dst: np.ndarray     #   first packed row of its 32
    tail_req: np.ndarray     # per request whose history ends mid-page: request,
    tail_info: np.ndarray    #   [first packed row, tokens, tail slot]
    new_dst: np.ndarray      # per new token, in the step's order: packed row


def pack_plan(new_tokens, history, slots) -> PackPlan:
    """The plan of consecutive requests with `new_tokens` queries over `history` cached tokens each,
    tails in request-pool `slots`."""
    q = np.asarray(new_tokens, dtype=np.int64)
    h = np.asarray(history, dtype=np.int64)
    slots = np.asarray(slots, dtype=np.int64)
    R = len(q)
    key_start = np.zeros(R + 1, dtype=np.int64)
    np.cumsum(h + q, out=key_start[1:])
    full, part = h // PAGE, h % PAGE
    page_req = np.repeat(np.arange(R), full)
    first_page = np.cumsum(full) - full
    page_index = np.arange(int(full.sum()), dtype=np.int64) - first_page[page_req]
    page_dst = key_start[page_req] + page_index * PAGE
    tail_req = np.flatnonzero(part)
    tail_info = np.stack([key_start[tail_req] + full[tail_req] * PAGE, part[tail_req], slots[tail_req]], axis=1)
    token_req = np.repeat(np.arange(R), q)
    first_token = np.cumsum(q) - q
    new_dst = key_start[token_req] + h[token_req] + np.arange(int(q.sum()), dtype=np.int64) - first_token[token_req]
    return PackPlan(key_start, page_req, page_index, page_dst, tail_req, tail_info.reshape(-1, 3), new_dst)


@dataclass
class Group:
    """Consecutive requests [r0, r1) of a step, attended together (packed) or one at a time."""
    r0: int
    r1: int
    packed: bool
    has_history: bool = False
    n_keys: int = 0
    key_start: list | None = None      # group-local, host
    max_q: int = 0
    max_k: int = 0
    cu_q: torch.Tensor | None = None   # int32 [rows + 1]: group-local query / key offsets, for varlen kernels
    cu_k: torch.Tensor | None = None
    page_blk: torch.Tensor | None = None
    page_dst: torch.Tensor | None = None
    tail_blk: torch.Tensor | None = None
    tail_info: torch.Tensor | None = None
    new_dst: torch.Tensor | None = None


def group_requests(new_tokens: np.ndarray, history: np.ndarray, bytes_per_key: int, budget: int, packed: bool):
    """[(r0, r1, packed)]: consecutive requests while their keys' K + V fit `budget`; a request over it
    alone, or every request when not `packed`, on its own with the history in blocks."""
    cost = (np.asarray(new_tokens, dtype=np.int64) + np.asarray(history, dtype=np.int64)) * bytes_per_key
    out, r, R = [], 0, len(cost)
    while r < R:
        if not packed or cost[r] > budget:
            out.append((r, r + 1, False))
            r += 1
            continue
        r1, used = r, 0
        while r1 < R and used + cost[r1] <= budget:
            used += int(cost[r1])
            r1 += 1
        out.append((r, r1, True))
        r = r1
    return out


def _host_to_device(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    return torch.from_numpy(arr).to(device)


@dataclass
class ExtendPlan:
    """The host plan and device index tensors of one extend step, shared by its layers. Built from
    the requests' new-token counts, cached history lengths and tail slots (host), and their block
    table (device int32 [R, pages])."""
    q_start: torch.Tensor                    # int32 [R + 1] query rows (device)
    job_seq: torch.Tensor                    # int32 write jobs: (request, logical page) per page touched
    job_page: torch.Tensor
    groups: list = field(default_factory=list)
    q_start_host: list = field(default_factory=list)
    history_host: list = field(default_factory=list)

    @classmethod
    def build(cls, new_tokens, history, slots, block_table: torch.Tensor, *, kv_heads: int, head_dim: int,
              dtype: torch.dtype, packed: bool = True, budget: int | None = None, upload=None) -> "ExtendPlan":
        """upload(int32 numpy array) -> device tensor: how the step's one host -> device copy is made
        (default: a plain copy to the block table's device)."""
        q = np.asarray(new_tokens, dtype=np.int64)
        h = np.asarray(history, dtype=np.int64)
        slots = np.asarray(slots, dtype=np.int64)
        total = h + q
        q_start = np.concatenate([[0], np.cumsum(q)])
        jobs = [(r, p) for r in range(len(q)) for p in pages_touched(int(h[r]), int(total[r]))]
        job_arr = np.asarray(jobs, dtype=np.int64).reshape(-1, 2)
        elem = torch.empty((), dtype=dtype).element_size()
        layout = group_requests(q, h, 2 * kv_heads * head_dim * elem, pack_budget() if budget is None else budget,
                                packed)
        host = [q_start, job_arr[:, 0], job_arr[:, 1]]
        plans = []
        for r0, r1, is_packed in layout:
            if not is_packed:
                plans.append(None)
                continue
            p = pack_plan(q[r0:r1], h[r0:r1], slots[r0:r1])
            plans.append(p)
            host += [p.key_start, q_start[r0:r1 + 1] - q_start[r0], r0 + p.page_req, p.page_index, p.page_dst,
                     r0 + p.tail_req, h[r0 + p.tail_req] // PAGE, p.tail_info.reshape(-1), p.new_dst]
        flat = np.concatenate(host).astype(np.int32)
        dev = (upload or (lambda a: _host_to_device(a, block_table.device)))(flat)
        views, at = [], 0
        for a in host:
            views.append(dev[at:at + len(a)])
            at += len(a)
        plan = cls(views[0], views[1], views[2], q_start_host=[int(x) for x in q_start],
                   history_host=[int(x) for x in h])
        rest = iter(views[3:])
        for (r0, r1, is_packed), p in zip(layout, plans):
            g = Group(r0, r1, is_packed)
            if p is not None:
                g.cu_k, g.cu_q, page_req, page_index, g.page_dst, tail_req, tail_page, g.tail_info, g.new_dst = (
                    next(rest) for _ in range(9))
                g.page_blk = block_table[page_req.long(), page_index.long()].contiguous()
                g.tail_blk = block_table[tail_req.long(), tail_page.long()].contiguous()
                g.key_start = [int(x) for x in p.key_start]
                g.n_keys = g.key_start[-1]
                g.has_history = bool(h[r0:r1].any())
                g.max_q = int(q[r0:r1].max())
                g.max_k = int(total[r0:r1].max())
            plan.groups.append(g)
        return plan

    def attend(self, ops, q3: torch.Tensor, k3: torch.Tensor, v3: torch.Tensor, cache: torch.Tensor,
               tail: torch.Tensor, block_table: torch.Tensor, slots: torch.Tensor, scale: float, rot: bool,
               out: torch.Tensor | None = None, varlen=None) -> torch.Tensor:
        """Attention of the step's queries q3 [T, Hq, D] (rows in request order) over each request's
        cached history and its new rows k3, v3 [T, Hk, D], reading the cache as it was before this
        step's write. varlen(q, k, v, group, scale, out): an optional varlen attention kernel for packed
        groups (causal, queries at the end of each request's keys); default: ragged_attention (torch's
        flash-attention kernel in its varlen form for bf16 / fp16 on the GPU)."""
        out = torch.empty(q3.shape, dtype=q3.dtype, device=q3.device) if out is None else out
        qs = self.q_start_host
        for g in self.groups:
            a, b = qs[g.r0], qs[g.r1]
            if b <= a:
                continue
            if g.packed:
                local = [x - a for x in qs[g.r0:g.r1 + 1]]
                if g.has_history:
                    kp = torch.empty((g.n_keys,) + tuple(k3.shape[1:]), dtype=k3.dtype, device=k3.device)
                    vp = torch.empty_like(kp)
                    if unpack_mode() == "torch":           # KUSHKASH_UNPACK=torch: the same bits, built by torch
                        torch_unpack(cache, g.page_blk, g.page_dst, g.tail_blk, g.tail_info, tail, k3[a:b], v3[a:b],
                                     g.new_dst, kp, vp, ops.D, ops.bits, rot)
                    else:
                        ops.unpack(cache, g.page_blk, g.page_dst, g.tail_blk, g.tail_info, tail, k3[a:b], v3[a:b],
                                   g.new_dst, kp, vp, rot)
                else:                                  # no history: the new rows are the keys
                    kp, vp = k3[a:b], v3[a:b]
                if varlen is not None:
                    varlen(q3[a:b], kp, vp, g, scale, out[a:b])
                else:
                    out[a:b] = ragged_attention(q3[a:b], kp, vp, local, g.key_start, scale,
                                                varlen=(g.cu_q, g.cu_k, g.max_q, g.max_k))
            else:
                r = g.r0

                def heads(x):
                    return x[a:b].transpose(0, 1).unsqueeze(0)         # [1, heads, T, D]
                o = unpacked_history_attention(ops, heads(q3), heads(k3), heads(v3), cache, block_table[r:r + 1],
                                               self.history_host[r], tail, slots[r:r + 1], scale, rot)
                out[a:b] = o[0].transpose(0, 1)
        return out

    def write(self, ops, k3: torch.Tensor, v3: torch.Tensor, seq_lens: torch.Tensor, slots: torch.Tensor,
              cache: torch.Tensor, block_table: torch.Tensor, tail: torch.Tensor, rot: bool) -> None:
        """Quantize the step's new rows into the cache (one write launch); seq_lens count them."""
        ops.write(k3, v3, self.q_start, seq_lens, slots, self.job_seq, self.job_page, cache, block_table, tail,
                  fused=True, rot=rot)
