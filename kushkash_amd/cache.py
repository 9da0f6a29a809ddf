"""KushCache: a paged int4 / int8 KV cache with fused decode attention, for a batch whose sequences
advance together (the Hugging Face integration and kushkash_amd.generate), on the gfx950 kernels of
Ops. Public API and semantics: the reference's KushCache and MemoryStats (kushkash/cache.py:43-246).

Storage
    pool         uint8 [L, blocks, Hkv, RB]   per layer, one record per (block, kv head)
    tail_k       [L, B, Hkv, 32, D]           per layer, the exact K of each sequence's partial page
                                              (kernel dtype); that page's V rows are final in its record
    seq_lens     int32 [L, B]                 per layer, tokens cached, on the device (kernels read it)
    block_table  int32 [B, pages]             shared by the layers: logical page -> block
    tail_idx     int32 [B]                    sequence b uses tail slot b

Page map. All sequences hold the same number of pages, so the map is a closed form: logical page p of
sequence b is block p * B + b. The B blocks of one logical page are adjacent (a chunk write's jobs
of one page touch neighbouring records), the table never changes once written, and growing the cache
only appends blocks: the pool is reallocated with the old blocks as its prefix.

Rotation. With rotation on (rotate=, KUSHKASH_ROTATE; on for 4-bit by default) the records and the
tail hold K H and V H for the Hadamard matrix H: K, V and q are rotated on the way in and the
decode output on the way out, by a torch product (the reference's rotation) or, with
rotate_in_kernels=True, inside the write, append and decode kernels. Every public method takes and
returns unrotated tensors.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from ._attention import unpacked_history_attention
from ._ops import PAGE, Ops, default_scale, pages_touched, record_bytes
from ._records import cached_kv
from ._rotation import hadamard, rotate, rotation_enabled

_KERNEL_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


@dataclass
class MemoryStats:
    """Bytes a KushCache holds (cache.py:23-40): its records in use, its exact K tails, what it has
    reserved, and what an fp16 cache of the same tokens would take."""
    tokens: int
    quantized_bytes: int
    tail_bytes: int
    reserved_bytes: int
    fp16_bytes: int

    @property
    def ratio(self) -> float:
        """fp16 bytes per byte in use (records + tails; the tails are a whole page per sequence and
        layer from the start, so short contexts compress less). int4 at D 128 tends to 3.46x."""
        used = self.quantized_bytes + self.tail_bytes
        return self.fp16_bytes / used if used else float("nan")


class KushCache:
    """
    Args:
        num_layers, num_kv_heads, num_q_heads, head_dim: the model's attention shape.
        batch_size: sequences per batch; they advance together.
        bits: 4 or 8.
        device: the ROCm device ("cuda[:i]"), or "cpu" for the host library (fp32 kernels and tails; q,
            k, v in `dtype` are converted), as the reference's CPU path.
        dtype: dtype of q, k, v handed in and of the attention output.
        max_length: per-sequence capacity to reserve up front (the pool grows on demand otherwise).
        scale: softmax scale (default 1 / sqrt(head_dim)).
        rotate: Hadamard rotation inside the cache; None reads KUSHKASH_ROTATE (auto: on for 4-bit).
        rotate_in_kernels: with rotation on, let the kernels rotate (canonical Walsh-Hadamard
            transform) instead of a torch product around them; no counterpart in the reference, the
            stored values differ from the product's only in rounding.
    """

    def __init__(self, num_layers: int, num_kv_heads: int, num_q_heads: int, head_dim: int, *,
                 batch_size: int = 1, bits: int = 4, device: str | torch.device = "cuda",
                 dtype: torch.dtype = torch.float16, max_length: int | None = None, scale: float | None = None,
                 rotate: bool | None = None, rotate_in_kernels: bool = False):
        if bits not in (4, 8):
            raise ValueError("bits must be 4 or 8")
        if num_kv_heads < 1 or num_q_heads % num_kv_heads:
            raise ValueError("num_q_heads must be a multiple of num_kv_heads")
        self.L, self.H, self.D, self.B = num_layers, num_kv_heads, head_dim, batch_size
        self.G = num_q_heads // num_kv_heads
        self.bits = bits
        self.RB = record_bytes(head_dim, bits)
        self.dtype = dtype
        self.scale = default_scale(head_dim) if scale is None else float(scale)
        device = torch.device(device)
        self.gpu = device.type == "cuda"
        if self.gpu:
            if dtype not in _KERNEL_DTYPES:
                raise ValueError(f"dtype must be one of {_KERNEL_DTYPES}")
            device = torch.device("cuda", torch.cuda.current_device() if device.index is None else device.index)
        self.device = device
        self.kdtype = dtype if self.gpu else torch.float32        # what the kernels and the tails hold
        self.ops = Ops(device, head_dim, bits, self.G, self.kdtype)
        self.rot = hadamard(head_dim, device) if rotation_enabled(bits, rotate) else None
        if rotate_in_kernels and not self.gpu:
            raise ValueError("rotate_in_kernels is for the GPU kernels; on the CPU the cache rotates with torch")
        self.krot = self.rot is not None and bool(rotate_in_kernels)
        self.profile: list | None = None                          # a list: attend_chunk records event pairs
        self.tail_k = torch.zeros(num_layers, batch_size, num_kv_heads, PAGE, head_dim, dtype=self.kdtype,
                                  device=device)
        self.tail_idx = torch.arange(batch_size, dtype=torch.int32, device=device)
        self.seq_lens = torch.zeros(num_layers, batch_size, dtype=torch.int32, device=device)
        self.pool = torch.zeros(num_layers, 0, num_kv_heads, self.RB, dtype=torch.uint8, device=device)
        self.block_table = torch.zeros(batch_size, 0, dtype=torch.int32, device=device)
        self._work = torch.zeros(0, dtype=torch.float32, device=device)
        self._tokens = [0] * num_layers                           # host copy of seq_lens (equal across the batch)
        self._splits = 0                                          # > 0 once freeze() fixed the split count
        self._capacity = 0
        self._reserve(-(-(max_length or 4 * PAGE) // PAGE))

    # ---------------------------------------------------------------- pages
    @property
    def pages(self) -> int:
        """Logical pages per sequence the pool holds."""
        return self.block_table.shape[1]

    def _reserve(self, pages: int) -> None:
        """Make room for `pages` logical pages per sequence: blocks [0, pages * B), the old ones kept in
        place, and the table's closed-form entries."""
        if pages <= self.pages:
            return
        if self._splits:
            raise RuntimeError(f"cache capacity {self._capacity} exceeded (set a larger max_length)")
        pages = max(pages, self.pages + self.pages // 2)
        old = self.pool
        self.pool = torch.zeros(self.L, pages * self.B, self.H, self.RB, dtype=torch.uint8, device=self.device)
        self.pool[:, :old.shape[1]] = old
        page = torch.arange(pages, dtype=torch.int32, device=self.device)
        seq = torch.arange(self.B, dtype=torch.int32, device=self.device)
        self.block_table = (page[None, :] * self.B + seq[:, None]).contiguous()

    def _ensure_work(self, splits: int) -> None:
        need = self.B * self.H * splits * self.G * (self.D + 2)
        if splits > 1 and self._work.numel() < need:
            self._work = torch.empty(need, dtype=torch.float32, device=self.device)

    # ---------------------------------------------------------------- rotation
    def _inward(self, x: torch.Tensor) -> torch.Tensor:
        """x in the kernel dtype, rotated by H unless the kernels rotate (or the cache does not)."""
        return x.to(self.kdtype) if self.krot or self.rot is None else rotate(x, self.rot, self.kdtype)

    def _outward(self, x: torch.Tensor) -> torch.Tensor:
        """A decode output of the kernels in the model dtype, rotated back unless the kernels did."""
        return x.to(self.dtype) if self.krot or self.rot is None else rotate(x, self.rot, self.dtype)

    def _unrotate(self, x: torch.Tensor) -> torch.Tensor:
        """Stored (rotated) values back in the model's basis, by the rotation that stored them: H is its
        own inverse, as a product or as the kernels' Walsh-Hadamard transform."""
        if self.rot is None:
            return x
        if not self.krot:
            return rotate(x, self.rot)
        y = self.ops.fwht(x.to(self.kdtype).reshape(-1, self.D).contiguous())
        return y.view(x.shape).to(x.dtype)

    def _rows(self, x: torch.Tensor) -> torch.Tensor:
        """[B, H, T, D] -> the kernels' rows [B * T, H, D] (head stride D) in the kernel dtype, rotated
        for a product-rotated cache. A model's K / V usually are a transpose of exactly that layout."""
        B, H, T, D = x.shape
        x = x.transpose(1, 2)
        if self.rot is not None and not self.krot:
            return rotate(x, self.rot, self.kdtype).view(B * T, H, D)
        x = x.to(self.kdtype)
        return (x if x.is_contiguous() else x.contiguous()).view(B * T, H, D)

    # ---------------------------------------------------------------- writes and attention
    def length(self, layer: int = 0) -> int:
        return self._tokens[layer]

    def write(self, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append T tokens to every sequence; k, v [B, Hkv, T, D]. One token takes the append kernel,
        which also counts it in seq_lens; a chunk takes the ragged write over every page it touches,
        seq_lens counting the chunk beforehand (cache.py:132-162)."""
        B, H, T, D = k.shape
        if (B, H, D) != (self.B, self.H, self.D) or v.shape != k.shape:
            raise ValueError(f"expected k, v of shape [{self.B}, {self.H}, T, {self.D}], got {tuple(k.shape)}")
        if T == 0:
            return
        n = self._tokens[layer]
        self._reserve(-(-(n + T) // PAGE))
        kw = {"rot": True} if self.krot else {}
        dst = dict(cache=self.pool[layer], block_table=self.block_table, tail_k=self.tail_k[layer])
        kr, vr = self._rows(k), self._rows(v)
        if T == 1:
            self.ops.append(kr, vr, self.seq_lens[layer], self.tail_idx, pos_offset=0, advance=True, **dst, **kw)
        else:
            self.seq_lens[layer].fill_(n + T)
            touched = pages_touched(n, n + T)
            pages = torch.arange(touched.start, touched.stop, dtype=torch.int32, device=self.device)
            seqs = torch.arange(B, dtype=torch.int32, device=self.device)
            starts = seqs * T
            qsl = torch.cat([starts, starts[-1:] + T])
            self.ops.write(kr, vr, qsl, self.seq_lens[layer], self.tail_idx,
                           seqs.repeat_interleave(len(touched)), pages.repeat(B), **dst, fused=True, **kw)
        self._tokens[layer] = n + T

    def attend(self, layer: int, q: torch.Tensor) -> torch.Tensor:
        """Decode attention of one query per sequence over all its cached tokens. q [B, Hq, D] (q head i
        reads kv head i // G); returns [B, Hq, D] in self.dtype (cache.py:164-183). Split-K partials
        go to a work buffer that only grows (freeze() sizes it for graph capture)."""
        if self._tokens[layer] == 0:
            raise RuntimeError("attend() on an empty cache")
        return self._decode(layer, q)

    def append_attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """write() of one token per sequence (k, v [B, Hkv, 1, D]) then attend(layer, q), the append done
        by the decode launch itself (Ops.append_decode): the same records, tails and output as the two
        calls, one launch fewer per decode step. No reference counterpart."""
        if k.shape != (self.B, self.H, 1, self.D) or v.shape != k.shape:
            raise ValueError(f"expected k, v of shape [{self.B}, {self.H}, 1, {self.D}], got {tuple(k.shape)}")
        n = self._tokens[layer]
        self._reserve(-(-(n + 1) // PAGE))
        token = (self._rows(k), self._rows(v))
        self.seq_lens[layer].add_(1)                     # the fused append writes at seq_lens - 1
        self._tokens[layer] = n + 1
        return self._decode(layer, q, token)

    def _decode(self, layer: int, q: torch.Tensor, token=None) -> torch.Tensor:
        qk = self._inward(q).contiguous()
        out = torch.empty_like(qk)
        pages = (self._capacity if self._splits else self._tokens[layer]) // PAGE
        splits = self._splits or self.ops.splits(self.B, self.H, pages)
        self._ensure_work(splits)
        kw = {"rot": True} if self.krot else {}
        if self.gpu:                                     # waves by the cached length (the table is wider)
            kw["waves"] = self.ops.waves(self.B, self.H, splits, pages)
        args = (self.pool[layer], self.block_table, self.seq_lens[layer], self.tail_idx, self.tail_k[layer],
                self.scale, splits, self._work)
        if token is None:
            self.ops.decode(qk, out, *args, **kw)
        else:
            self.ops.append_decode(token[0], token[1], qk, out, *args, **kw)
        return self._outward(out)

    def attend_chunk(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     block_bytes: int = 1 << 28) -> torch.Tensor:
        """Attention of a chunk of T queries over the cached history plus the chunk itself (causal),
        before the chunk is written; q [B, Hq, T, D], k, v [B, Hkv, T, D] -> [B, Hq, T, D]
        (cache.py:185-201). The history is unpacked a block of pages at a time by the unpack kernel,
        rotated back in that kernel when the cache rotates, so the attention itself runs on the
        unrotated q and chunk; extra memory stays within ~block_bytes at any history length."""
        timing = self.profile is not None and q.is_cuda
        if timing:
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        out = unpacked_history_attention(self.ops, q, k, v, self.pool[layer], self.block_table, self._tokens[layer],
                                         self.tail_k[layer], self.tail_idx, self.scale, self.rot is not None,
                                         block_bytes)
        if timing:
            ev[1].record()
            self.profile.append(ev)
        return out

    def dequantize(self, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Reference view: the cached K, V of `layer` as [B, Hkv, n, D] in self.dtype, dequantized by
        torch and rotated back; materializes the whole history (cache.py:203-208). Testing only."""
        k, v = cached_kv(self.pool[layer], self.block_table, self._tokens[layer], self.tail_k[layer], self.D,
                         self.bits, self.dtype)
        return self._unrotate(k), self._unrotate(v)

    # ---------------------------------------------------------------- graph capture
    def freeze(self, max_tokens: int) -> None:
        """Reserve pages for max_tokens per sequence and fix the split count, so that decode steps
        allocate nothing and can be captured in a HIP graph (cache.py:211-221)."""
        if not self.gpu:
            raise RuntimeError("freeze() is for the GPU path")
        self._reserve(-(-max_tokens // PAGE))
        self._splits = self.ops.splits(self.B, self.H, max_tokens // PAGE)
        self._ensure_work(self._splits)
        self._capacity = max_tokens

    def advance(self, steps: int = 1) -> None:
        """Count `steps` replayed decode steps on the host (inside the graph the append kernel counts
        them on the device)."""
        if max(self._tokens) + steps > self._capacity:
            raise RuntimeError(f"cache capacity {self._capacity} exceeded")
        self._tokens = [n + steps for n in self._tokens]

    def lengths(self) -> list[int]:
        """The host-side token counts of every layer (a copy)."""
        return list(self._tokens)

    def set_lengths(self, tokens: list[int]) -> None:
        """Restore host-side token counts taken by lengths() (a graph capture records calls without
        running them)."""
        if len(tokens) != self.L:
            raise ValueError(f"expected {self.L} lengths")
        self._tokens = [int(n) for n in tokens]

    def reset(self) -> None:
        """Drop every token; the pool, table and tails stay allocated, and the split count is free again."""
        self._tokens = [0] * self.L
        self.seq_lens.zero_()
        self._splits = 0
        self._capacity = 0

    def memory(self) -> MemoryStats:
        n = max(self._tokens)
        tails = self.tail_k.numel() * self.tail_k.element_size()
        return MemoryStats(tokens=n, quantized_bytes=self.L * self.B * self.H * -(-n // PAGE) * self.RB,
                           tail_bytes=tails, reserved_bytes=self.pool.numel() + tails,
                           fp16_bytes=2 * self.L * self.B * self.H * n * self.D * 2)
