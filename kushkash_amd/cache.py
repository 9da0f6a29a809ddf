"""KushCache: paged, quantized KV cache (int4 / int8) with fused decode attention, for equal-length
batches. Same public API as the reference's ``kushkash/cache.py`` (KushCache, MemoryStats); the
kernels behind it are the gfx950 HIP kernels of ``Ops``.

Memory per layer
    pool     uint8 [pages, Hkv, RB]       one record per (page, kv head): codes + scales
    tail_k   [B, Hkv, 32, D]              K of the page being filled, exact (model dtype); its V rows
                                          are already final in the page's record
Shared by all layers: block_table int32 [B, max_pages] (logical -> physical page).
With rotation on (rotate=, KUSHKASH_ROTATE) pages and tail hold K H and V H (Hadamard H); every
public method takes and returns unrotated tensors. The rotation is the reference's GEMM by default;
rotate_in_kernels=True folds it into the kernels instead (the canonical Walsh-Hadamard transform
inside the write, append and decode launches: no rotation GEMMs per step).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ._ops import (PAGE, Ops, as_records, cached_kv, default_scale, hadamard, history_attention, record_bytes,
                   rotate, rotation_enabled)

_GPU_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


@dataclass
class MemoryStats:
    tokens: int            # tokens cached per sequence
    quantized_bytes: int   # page records in use, all layers
    tail_bytes: int        # exact K tails, all layers
    reserved_bytes: int    # pool capacity incl. unused pages
    fp16_bytes: int        # what an fp16 cache of the same content would take

    @property
    def ratio(self) -> float:
        """fp16 bytes / bytes used, including the exact K tails (cache.py:34-40)."""
        used = self.quantized_bytes + self.tail_bytes
        return self.fp16_bytes / used if used else float("nan")


class KushCache:
    """
    Args:
        num_layers, num_kv_heads, num_q_heads, head_dim: model attention shape.
        batch_size: sequences per batch (they advance together).
        bits: 4 or 8.
        device: "cuda[:i]" (the ROCm device).
        dtype: dtype of q / k / v given to the cache and of the attention output.
        max_length: optional per-sequence capacity hint; pools grow on demand otherwise.
        scale: softmax scale (default 1/sqrt(head_dim)).
        rotate: Hadamard-rotate K, V and q inside the cache. None: KUSHKASH_ROTATE (auto: on for
            4-bit, off for 8-bit). Inputs and outputs stay unrotated.
        rotate_in_kernels: with rotation on, rotate inside the kernels (canonical Walsh-Hadamard
            transform, as Ops.fwht) instead of with a GEMM before and after them. No counterpart in
            the reference; the rotated values differ from the GEMM's only in rounding.
    Contract: kushkash/cache.py:43-246.
    """

    def __init__(self, num_layers: int, num_kv_heads: int, num_q_heads: int, head_dim: int, *,
                 batch_size: int = 1, bits: int = 4, device: str | torch.device = "cuda",
                 dtype: torch.dtype = torch.float16, max_length: int | None = None, scale: float | None = None,
                 rotate: bool | None = None, rotate_in_kernels: bool = False):
        if bits not in (4, 8):
            raise ValueError("bits must be 4 or 8")
        if num_q_heads % num_kv_heads:
            raise ValueError("num_q_heads must be a multiple of num_kv_heads")
        self.L, self.H, self.D, self.B = num_layers, num_kv_heads, head_dim, batch_size
        self.G = num_q_heads // num_kv_heads
        self.bits = bits
        self.RB = record_bytes(head_dim, bits)
        self.device = torch.device(device)
        self.dtype = dtype
        self.scale = float(scale) if scale is not None else default_scale(head_dim)
        self.gpu = self.device.type == "cuda"
        if self.gpu:
            if dtype not in _GPU_DTYPES:
                raise ValueError(f"dtype must be one of {_GPU_DTYPES}")
            if self.device.index is None:
                self.device = torch.device("cuda", torch.cuda.current_device())
        self.kdtype = dtype if self.gpu else torch.float32            # kernel / tail dtype
        self.ops = Ops(self.device, head_dim, bits, self.G, self.kdtype)
        self.rot = hadamard(head_dim, self.device) if rotation_enabled(bits, rotate) else None
        self.krot = bool(rotate_in_kernels) and self.rot is not None      # rotation folded into the kernels
        self._work = torch.empty(0, dtype=torch.float32, device=self.device)
        pages0 = max(1, -(-(max_length or 4 * PAGE) // PAGE))
        self._pages = 0
        self.pool = torch.empty(0, dtype=torch.uint8, device=self.device)
        self._alloc_pages(batch_size * pages0)
        self.block_table = torch.zeros(batch_size, pages0, dtype=torch.int32, device=self.device)
        self.tail_k = torch.zeros(num_layers, batch_size, num_kv_heads, PAGE, head_dim, dtype=self.kdtype,
                                  device=self.device)
        self.tail_idx = torch.arange(batch_size, dtype=torch.int32, device=self.device)
        self.seq_lens = torch.zeros(num_layers, batch_size, dtype=torch.int32, device=self.device)
        self._len = [0] * num_layers            # host mirror of seq_lens (all sequences equal)
        self._mapped = 0                        # logical pages mapped per sequence
        self._next = 0                          # bump allocator over physical pages
        self._frozen_ns = 0                     # split-K fixed by freeze() (graph capture)
        self._capacity = 0
        self.profile: list | None = None        # set to [] to record attend_chunk events

    # ---------------------------------------------------------------- page management
    def _alloc_pages(self, n: int) -> None:
        """(Re)allocate the pool for n physical pages, keeping the existing ones."""
        new = torch.zeros(self.L, n, self.H, self.RB, dtype=torch.uint8, device=self.device)
        if self._pages:
            new[:, :self._pages] = self.pool
        self.pool, self._pages = new, n

    def _map(self, need: int) -> None:
        """Map logical pages [0, need) of every sequence to physical pages from a bump allocator;
        pages are never freed before reset(), so table entries stay valid (cache.py:106-126)."""
        if need <= self._mapped:
            return
        if self._frozen_ns:
            raise RuntimeError(f"cache capacity {self._capacity} exceeded (set a larger max_length)")
        add = need - self._mapped
        if self._next + add * self.B > self._pages:
            self._alloc_pages(max(2 * self._pages, self._next + add * self.B))
        if need > self.block_table.shape[1]:
            bt = torch.zeros(self.B, max(need, 2 * self.block_table.shape[1]), dtype=torch.int32, device=self.device)
            bt[:, :self.block_table.shape[1]] = self.block_table
            self.block_table = bt
        ids = torch.arange(self._next, self._next + add * self.B, dtype=torch.int32, device=self.device)
        self.block_table[:, self._mapped:need] = ids.view(self.B, add)
        self._next += add * self.B
        self._mapped = need

    # ---------------------------------------------------------------- public API
    def length(self, layer: int = 0) -> int:
        return self._len[layer]

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append T new tokens for every sequence. k, v: [B, Hkv, T, D]. T == 1 takes the append
        kernel (which advances seq_lens itself); a longer chunk takes the ragged write with one job
        per (sequence, logical page) touched, seq_lens already counting the new tokens
        (cache.py:132-162)."""
        B, H, T, D = k.shape
        if (B, H, D) != (self.B, self.H, self.D) or v.shape != k.shape:
            raise ValueError(f"expected k, v of shape [{self.B}, {self.H}, T, {self.D}], got {tuple(k.shape)}")
        if T == 0:
            return
        n = self._len[layer]
        self._map(-(-(n + T) // PAGE))                 # incl. the partial page (it holds its V rows)
        if not self.krot:
            k, v = rotate(k, self.rot, self.kdtype), rotate(v, self.rot, self.kdtype)
        k = k.transpose(1, 2).to(self.kdtype)          # kernel rows: [B*T, H, D], head stride D
        v = v.transpose(1, 2).to(self.kdtype)
        if k.stride(-1) != 1 or k.stride(-2) != D or k.stride(0) != T * k.stride(1) or v.stride() != k.stride():
            k, v = k.contiguous(), v.contiguous()
        k, v = k.reshape(B * T, H, D), v.reshape(B * T, H, D)
        args = dict(cache=self.pool[layer], block_table=self.block_table, tail_k=self.tail_k[layer])
        if self.krot:
            args["rot"] = True
        if T == 1:
            self.ops.append(k, v, self.seq_lens[layer], self.tail_idx, pos_offset=0, advance=True, **args)
        else:
            self.seq_lens[layer].fill_(n + T)
            pages = torch.arange(n // PAGE, (n + T - 1) // PAGE + 1, dtype=torch.int32, device=self.device)
            job_seq = torch.arange(B, dtype=torch.int32, device=self.device).repeat_interleave(pages.numel())
            qsl = torch.arange(B + 1, dtype=torch.int32, device=self.device) * T
            self.ops.write(k, v, qsl, self.seq_lens[layer], self.tail_idx, job_seq, pages.repeat(B), **args)
        self._len[layer] = n + T

    def attend(self, layer: int, q: torch.Tensor) -> torch.Tensor:
        """Decode attention of one query token per sequence over the whole cache. q: [B, Hq, D]
        (q head i uses kv head i // G); returns [B, Hq, D] in self.dtype. Split-K partials go to
        `_work` (only grows; freeze() fixes it for graph capture) (cache.py:164-183)."""
        if self._len[layer] == 0:
            raise RuntimeError("attend() on an empty cache")
        return self._decode(layer, q, None, None)

    def append_attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """write(layer, k, v) of one token per sequence, then attend(layer, q), with the append done
        inside the decode launch (Ops.append_decode): one launch fewer per decode step. k, v: [B, Hkv,
        1, D]; q: [B, Hq, D]. The same cache contents and outputs as the two calls. No reference
        counterpart (its attention backends call write, then attend)."""
        B, H, T, D = k.shape
        if (B, H, T, D) != (self.B, self.H, 1, self.D) or v.shape != k.shape:
            raise ValueError(f"expected k, v of shape [{self.B}, {self.H}, 1, {self.D}], got {tuple(k.shape)}")
        n = self._len[layer]
        self._map(-(-(n + 1) // PAGE))
        if not self.krot:
            k, v = rotate(k, self.rot, self.kdtype), rotate(v, self.rot, self.kdtype)
        k = k.to(self.kdtype).reshape(B, H, D).contiguous()
        v = v.to(self.kdtype).reshape(B, H, D).contiguous()
        self.seq_lens[layer].add_(1)                   # the kernel appends at seq_lens - 1 (counted)
        self._len[layer] = n + 1
        return self._decode(layer, q, k, v)

    def _decode(self, layer: int, q: torch.Tensor, k: torch.Tensor | None, v: torch.Tensor | None) -> torch.Tensor:
        q = (q.to(self.kdtype) if self.krot else rotate(q, self.rot, self.kdtype)).contiguous()
        out = torch.empty_like(q)
        pages = (self._capacity if self._frozen_ns else self._len[layer]) // PAGE
        ns = self._frozen_ns or self.ops.splits(self.B, self.H, pages)
        if ns > 1:
            need = self.B * self.H * ns * self.G * (2 + self.D)
            if self._work.numel() < need:
                self._work = torch.empty(need, dtype=torch.float32, device=self.device)
        # GPU: the waves per workgroup from the cached length (the block table may be wider)
        kw = {"waves": self.ops.waves(self.B, self.H, ns, pages)} if self.gpu else {}
        if self.krot:
            kw["rot"] = True
        args = (self.pool[layer], self.block_table, self.seq_lens[layer], self.tail_idx, self.tail_k[layer], self.scale,
                ns, self._work)
        if k is None:
            self.ops.decode(q, out, *args, **kw)
        else:
            self.ops.append_decode(k, v, q, out, *args, **kw)
        return out.to(self.dtype) if self.krot else rotate(out, self.rot, self.dtype)

    def attend_chunk(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     block_bytes: int = 1 << 28) -> torch.Tensor:
        """Attention of a chunk of T queries over the cached history plus the chunk itself (causal),
        before the chunk is written. q: [B, Hq, T, D]; k, v: [B, Hkv, T, D] (cache.py:185-201)."""
        prof = self.profile is not None and q.is_cuda
        if prof:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        q, k, v = self._rotate(q), self._rotate(k), self._rotate(v)
        out = history_attention(q, k, v, as_records(self.pool[layer]), self.block_table, self._len[layer],
                                self.tail_k[layer], self.D, self.bits, self.scale, block_bytes)
        out = self._rotate(out)
        if prof:
            ev[1].record()
            self.profile.append(ev)
        return out

    def dequantize(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Reference: the cached K, V of `layer` as [B, Hkv, n, D] in self.dtype, rotated back if the
        cache rotates. Testing only (cache.py:203-208)."""
        k, v = cached_kv(self.pool[layer], self.block_table, self._len[layer], self.tail_k[layer], self.D,
                         self.bits, self.dtype)
        return self._rotate(k), self._rotate(v)

    def _rotate(self, x: torch.Tensor) -> torch.Tensor:
        """x rotated (or rotated back: the rotation is its own inverse) the way the cache's contents are:
        the reference's GEMM, or with rotate_in_kernels the kernels' Walsh-Hadamard transform."""
        if not self.krot:
            return rotate(x, self.rot)
        y = self.ops.fwht(x.to(self.kdtype).reshape(-1, self.D).contiguous())
        return y.view(x.shape).to(x.dtype)

    # ---------------------------------------------------------------- graph-capture support
    def freeze(self, max_tokens: int) -> None:
        """Pre-map pages for `max_tokens` per sequence and fix the split-K factor, so decode steps
        allocate nothing on the host and can be captured in a HIP graph (cache.py:211-221)."""
        if not self.gpu:
            raise RuntimeError("freeze() is for the GPU path")
        self._map(-(-max_tokens // PAGE))
        self._frozen_ns = self.ops.splits(self.B, self.H, max_tokens // PAGE)
        need = self.B * self.H * self._frozen_ns * self.G * (2 + self.D)
        if self._work.numel() < need:
            self._work = torch.empty(need, dtype=torch.float32, device=self.device)
        self._capacity = max_tokens

    def advance(self, steps: int = 1) -> None:
        """Host bookkeeping after replaying `steps` captured decode steps (the append kernel inside
        the graph advances the device seq_lens)."""
        if max(self._len) + steps > self._capacity:
            raise RuntimeError(f"cache capacity {self._capacity} exceeded")
        self._len = [n + steps for n in self._len]

    def reset(self) -> None:
        """Drop all tokens (keeps the allocated pools)."""
        self._len = [0] * self.L
        self.seq_lens.zero_()
        self._mapped = 0
        self._next = 0
        self._frozen_ns = 0

    def memory(self) -> MemoryStats:
        n = max(self._len)
        return MemoryStats(
            tokens=n,
            quantized_bytes=self.L * self.B * -(-n // PAGE) * self.H * self.RB,
            tail_bytes=self.tail_k.numel() * self.tail_k.element_size(),
            reserved_bytes=self.pool.numel() + self.tail_k.numel() * self.tail_k.element_size(),
            fp16_bytes=self.L * self.B * self.H * n * self.D * 2 * 2,
        )
