"""Kernel launcher over the page-record layout, and the pure-torch helpers around it.

Drop-in for the reference's ``kushkash/_ops.py``: ``Ops`` keeps its constructor, method names,
argument meaning and error behaviour (``_ops.py:42-213``). On a ROCm device every method runs a
hand-written gfx950 HIP kernel through the C ABI of ``libkushhip.so`` (include/kushkash_amd.h) on
torch's current stream; on device "cpu" it runs the host library ``libkushcpu.so`` (csrc/kush_cpu.cpp,
the reference's CPU library's C ABI), fp32 tensors only, as the reference's CPU path. The reference's torch helpers (record dequantization, attention with log-sum-exp,
rotation) are importable from here under their reference names; they live in _records, _attention
and _rotation.

Tensor conventions (as the reference, ``_ops.py:6-15``)
  cache       any tensor whose dim 0 is the block and dim 1 the kv head, each (block, head) record
              contiguous: uint8 [pages, H, RB], or a vLLM-style [blocks, H, 32, C] view
  tail_k      [slots, H, 32, D] in the kernel dtype: K of the page being filled, exact; sequence s
              uses slot tail_idx[s]; its V rows are already final in the page's record
  k, v rows   [rows, H, D] (row strides free, may differ between k and v; head stride D)
  q, out      [S, Hq, D] contiguous
  rotation    append / write / decode do not rotate: callers pass q H, k H, v H (rotate(), or
              Ops.fwht in the kernels' canonical order) and rotate back; unpack can rotate history back

"""
from __future__ import annotations

import math
import os
from dataclasses import dataclass

import torch

PAGE = 32
DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
DECODE_WAVES = 4                # default waves per decode workgroup (kush_decode: waves = 0)
SYNC_SLOTS = 1 << 16            # split-K merge counters per Ops: (sequence, kv head, 16-head chunk) slots


def record_bytes(head_dim: int, bits: int) -> int:
    """Bytes of one (page, kv head) record: 32 K rows + 32 V rows of codes, then fp16 K scale and bias
    per channel and fp16 V scale and bias per token (quant.mojo:60-61)."""
    row = head_dim if bits == 8 else head_dim // 2
    return 2 * PAGE * row + 4 * head_dim + 4 * PAGE


def _byte_strides(cache: torch.Tensor) -> tuple[int, int]:
    """Block and head strides in bytes: a cache can be a strided slice of a larger allocation
    (vLLM's), so the strides need not be the packed ones (_ops.py:34-39)."""
    e = cache.element_size()
    return cache.stride(0) * e, cache.stride(1) * e


@dataclass(frozen=True)
class KernelConfig:
    """What the reference exposes as ``Ops.cfg`` (its GpuConfig, _build.py:112-149), for callers
    that print or branch on it. Every decode here runs on the matrix cores (MFMA)."""
    head_dim: int
    bits: int
    group: int
    dtype: str
    arch: str = "gfx950"
    tensor_cores: bool = True
    warps: int = DECODE_WAVES

    def kernels(self) -> dict[str, str]:
        D, B, G, IN = self.head_dim, self.bits, self.group, self.dtype
        return {"append": f"append_kernel<{D},{B},{IN}>", "write": f"write_kernel<{D},{B},{IN}>",
                "decode": f"decode_kernel<{D},{B},{IN},{self.warps}> (group {G})", "combine": f"combine_kernel<{IN}>",
                "fwht": f"fwht_kernel<{D},{IN}>", "unpack": f"unpack_kernel<{D},{B},{IN}>"}


def _require(ok: bool, message: str) -> None:
    """The reference's argument errors are ValueErrors (_ops.py:109-168)."""
    if not ok:
        raise ValueError(message)


def _validate_default() -> bool:
    return os.environ.get("KUSHKASH_AMD_VALIDATE", "0") not in ("", "0")


def check_unpack_indices(page_blk: torch.Tensor, page_dst: torch.Tensor, tail_blk: torch.Tensor,
                         tail_info: torch.Tensor, new_dst: torch.Tensor, rows: int, blocks: int, slots: int) -> None:
    """Ops.unpack's index ranges (the reference checks them on its CPU path, _ops.py:153-164; the
    kernel trusts them): kp rows, cache blocks, tail slots and 1..32 tokens per partial page.
    Raises ValueError naming the offending indices. Reads the values, so on GPU tensors it
    synchronizes (Ops.validate)."""
    def outside(t: torch.Tensor, lo: int, hi: int) -> bool:        # a value outside [lo, hi)
        return t.numel() > 0 and (int(t.min()) < lo or int(t.max()) >= hi)

    first, tokens, slot = tail_info.view(-1, 3).long().unbind(1)
    checks = {"page_blk": outside(page_blk, 0, blocks), "tail_blk": outside(tail_blk, 0, blocks),
              "page_dst": outside(page_dst, 0, rows - PAGE + 1), "new_dst": outside(new_dst, 0, rows),
              "tail_info tokens": outside(tokens, 1, PAGE + 1), "tail_info slot": outside(slot, 0, slots),
              "tail_info rows": outside(first, 0, rows) or outside(first + tokens, 1, rows + 1)}
    bad = [name for name, hit in checks.items() if hit]
    if bad:
        raise ValueError(f"unpack: index out of range: {', '.join(bad)} "
                         f"({rows} rows, {blocks} blocks, {slots} tail slots, 1..{PAGE} tokens per partial page)")


class Ops:
    """Kernels for one (device, head_dim, bits, q heads per kv head, dtype): the gfx950 library on a
    ROCm device, the host library on device "cpu" (fp32; the reference's CPU path, _ops.py:49-57)."""

    def __init__(self, device: torch.device, head_dim: int, bits: int, group: int, dtype: torch.dtype,
                 *, validate: bool | None = None):
        device = torch.device(device)
        if device.type not in ("cuda", "cpu"):
            raise ValueError("kushkash_amd runs on the GPU (device 'cuda' under ROCm) or on the host (device 'cpu')")
        where = "GPU" if device.type == "cuda" else "CPU"
        if head_dim not in (64, 128, 256):
            raise ValueError(f"{where} head_dim must be 64, 128 or 256")
        if bits not in (4, 8):
            raise ValueError("bits must be 4 or 8")
        if group < 1:
            raise ValueError("group must be >= 1")
        if dtype not in DTYPE_CODE:
            raise ValueError(f"dtype must be one of {tuple(DTYPE_CODE)}")
        self.D, self.bits, self.G, self.dtype = head_dim, bits, group, dtype
        self.validate = _validate_default() if validate is None else validate
        self._dt = DTYPE_CODE[dtype]
        if device.type == "cpu":
            if dtype != torch.float32:
                raise ValueError("the CPU path computes in fp32: its tensors (and dtype) are torch.float32")
            from . import _cpu
            self._cpu = _cpu
            _cpu.lib()                                          # fail loudly now if it is not built
            self.device, self.gpu, self.sms = torch.device("cpu"), False, 1
            self.cfg = KernelConfig(head_dim, bits, group, "float32", arch="cpu", tensor_cores=False, warps=1)
            return
        from . import _lib
        self._lib = _lib
        _lib.lib()                                              # fail loudly now if it is not built
        idx = device.index if device.index is not None else torch.cuda.current_device()
        self.device = torch.device("cuda", idx)
        self.gpu = True
        self.sms = torch.cuda.get_device_properties(idx).multi_processor_count
        self.cfg = KernelConfig(head_dim, bits, group, str(dtype).split(".")[1])
        # counters of the fused split-K merge: zero at rest (the last workgroup of each (sequence, kv
        # head) resets its own), so one buffer serves every call of this Ops on one stream at a time
        self._sync = torch.zeros(SYNC_SLOTS, dtype=torch.int32, device=self.device)

    # ---------------------------------------------------------------- argument checks
    def _validating(self) -> bool:
        """Whether to check index values (validate on, and the stream not capturing a graph: the
        checks read values back to the host, which a capture does not allow)."""
        return self.validate and (not self.gpu or not torch.cuda.is_current_stream_capturing())

    def _stream(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _on_device(self, **ts: torch.Tensor) -> None:
        for name, t in ts.items():
            if t.device != self.device:
                raise ValueError(f"{name} is on {t.device}, these kernels run on {self.device}")

    def _check_index(self, **ts: torch.Tensor) -> None:
        for name, t in ts.items():
            if t.dtype != torch.int32 or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous int32 tensor")

    def _check_rows(self, name: str, t: torch.Tensor, H: int) -> None:
        if t.dim() != 3 or t.shape[1] != H or t.shape[2] != self.D or t.stride(2) != 1 or t.stride(1) != self.D:
            raise ValueError(f"{name} must be [rows, {H}, {self.D}] with unit dim stride and head stride {self.D}")
        if t.dtype != self.dtype:
            raise ValueError(f"{name} is {t.dtype}, these kernels take {self.dtype}")

    def _check_cache(self, cache: torch.Tensor, block_table: torch.Tensor, tail_k: torch.Tensor, H: int) -> None:
        bs, hs = _byte_strides(cache)
        if cache.dim() < 2 or cache.shape[1] < H:
            raise ValueError("cache must be [blocks, >= Hkv, ...]")
        if (cache.data_ptr() | bs | hs) % 16:
            raise ValueError("cache records must be 16-byte aligned (pointer, block and head strides)")
        if tail_k.dim() != 4 or tail_k.shape[1:] != (H, PAGE, self.D) or not tail_k.is_contiguous():
            raise ValueError(f"tail_k must be contiguous [slots, {H}, {PAGE}, {self.D}]")
        if tail_k.dtype != self.dtype:
            raise ValueError(f"tail_k is {tail_k.dtype}, these kernels take {self.dtype}")
        if block_table.dim() != 2 or block_table.dtype != torch.int32 or block_table.stride(1) != 1:
            raise ValueError("block_table must be int32 [S, max_pages] with unit column stride")

    def _check_values(self, cache, block_table, seq_lens, tail_idx, tail_k, rows: int, extra: int = 0) -> None:
        """Index ranges (one host sync; on when validate=True or KUSHKASH_AMD_VALIDATE=1): the kernels
        themselves do no bounds checks, as the reference's. extra: tokens added to seq_lens before the
        pages are counted (append: pos_offset + 1; rows left at <= 0 tokens are padding)."""
        if rows == 0 or not self._validating():
            return
        lens = (seq_lens[:rows].long() + extra).clamp(min=0)
        pages = (lens + PAGE - 1) // PAGE
        need = int(pages.max())
        if need > block_table.shape[1]:
            raise ValueError(f"block_table has {block_table.shape[1]} pages per sequence, {need} needed")
        if need:
            used = torch.arange(need, device=block_table.device)[None, :] < pages[:, None]
            ids = block_table[:rows, :need][used]
            if ids.numel() and (int(ids.min()) < 0 or int(ids.max()) >= cache.shape[0]):
                raise ValueError(f"block_table points outside the cache ({cache.shape[0]} blocks)")
        ti = tail_idx[:rows]
        if int(ti.min()) < 0 or int(ti.max()) >= tail_k.shape[0]:
            raise ValueError("tail_idx points outside tail_k")

    # ---------------------------------------------------------------- writes
    def append(self, k: torch.Tensor, v: torch.Tensor, seq_lens: torch.Tensor, tail_idx: torch.Tensor,
               cache: torch.Tensor, block_table: torch.Tensor, tail_k: torch.Tensor,
               pos_offset: int, advance: bool, *, rot: bool = False) -> None:
        """One token per sequence: row s of k/v goes to position seq_lens[s] + pos_offset (_ops.py:66-80).
        rot: rotate the rows by the canonical Walsh-Hadamard transform (rounded to the dtype, as fwht)
        inside the kernel before they are stored (no reference counterpart: its caches rotate with a GEMM)."""
        S, H = k.shape[0], k.shape[1]
        self._check_rows("k", k, H)
        self._check_rows("v", v, H)
        if v.shape[0] < S:
            raise ValueError("v must hold one row per sequence")
        self._check_index(seq_lens=seq_lens, tail_idx=tail_idx)
        self._check_cache(cache, block_table, tail_k, H)
        self._on_device(k=k, v=v, seq_lens=seq_lens, tail_idx=tail_idx, cache=cache, block_table=block_table,
                        tail_k=tail_k)
        if seq_lens.numel() < S or tail_idx.numel() < S or block_table.shape[0] < S:
            raise ValueError("seq_lens, tail_idx and block_table need one entry per sequence")
        self._check_values(cache, block_table, seq_lens, tail_idx, tail_k, S, extra=pos_offset + 1)
        bs, hs = _byte_strides(cache)
        if not self.gpu:
            _require(not rot, "append(rot=True) is a GPU extension; the CPU path takes rotated rows (fwht)")
            self._cpu.call("kush_cpu_append", self.D, self.bits, k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0),
                           seq_lens.data_ptr(), int(pos_offset), int(bool(advance)), cache.data_ptr(), bs, hs,
                           tail_k.data_ptr(), tail_idx.data_ptr(), block_table.data_ptr(), block_table.stride(0), H, S)
            return
        self._lib.call("kush_append_ex", self.D, self.bits, self._dt, k.data_ptr(), v.data_ptr(), k.stride(0),
                       v.stride(0), seq_lens.data_ptr(), int(pos_offset), int(bool(advance)), tail_idx.data_ptr(),
                       cache.data_ptr(), bs, hs, tail_k.data_ptr(), block_table.data_ptr(), block_table.stride(0),
                       H, S, self._stream(), int(bool(rot)))

    def write(self, k: torch.Tensor, v: torch.Tensor, query_start_loc: torch.Tensor, seq_lens: torch.Tensor,
              tail_idx: torch.Tensor, job_seq: torch.Tensor, job_page: torch.Tensor, cache: torch.Tensor,
              block_table: torch.Tensor, tail_k: torch.Tensor, *, fused: bool = False, rot: bool = False) -> None:
        """Ragged multi-token write: sequence s owns rows [qsl[s], qsl[s+1]) at positions ending at
        seq_lens[s] (already counting them); one job per (sequence, logical page) touched
        (_ops.py:82-101). By default the reference's two ordered launches (mode 0: V rows + completed
        K pages, then mode 1: K tails), which accept any subset of those jobs. fused=True declares that
        the list holds a job for every page each chunk touches (pages_touched, as this package's callers
        build it) and runs both modes as one launch (mode 2), whose tail handling relies on that; under
        KUSHKASH_AMD_VALIDATE the declaration is checked and a list that misses a touched page raises.
        rot: as in append (rows from the chunk are rotated)."""
        n_jobs, H = job_seq.numel(), k.shape[1]
        if n_jobs == 0:
            return
        self._check_rows("k", k, H)
        self._check_rows("v", v, H)
        self._check_index(query_start_loc=query_start_loc, seq_lens=seq_lens, tail_idx=tail_idx, job_seq=job_seq,
                          job_page=job_page)
        if job_page.numel() != n_jobs:
            raise ValueError("job_seq and job_page must have the same length")
        self._check_cache(cache, block_table, tail_k, H)
        self._on_device(k=k, v=v, query_start_loc=query_start_loc, seq_lens=seq_lens, tail_idx=tail_idx,
                        job_seq=job_seq, job_page=job_page, cache=cache, block_table=block_table, tail_k=tail_k)
        if self._validating():
            S = seq_lens.numel()
            js = job_seq.long()
            if int(js.min()) < 0 or int(js.max()) >= S or query_start_loc.numel() < S + 1:
                raise ValueError("job_seq points outside the batch")
            if int(query_start_loc[-1]) > min(k.shape[0], v.shape[0]):
                raise ValueError("query_start_loc points past the k / v rows")
            pages = (seq_lens.long()[js] + PAGE - 1) // PAGE
            if bool((job_page.long() < 0).any()) or bool((job_page.long() >= pages).any()):
                raise ValueError("job_page outside the sequence's pages")
            if fused:
                _check_covers(query_start_loc, seq_lens, job_seq, job_page)
            self._check_values(cache, block_table, seq_lens, tail_idx, tail_k, S)
        bs, hs = _byte_strides(cache)
        if not self.gpu:                                         # the two modes, in order, on the host
            _require(not rot, "write(rot=True) is a GPU extension; the CPU path takes rotated rows (fwht)")
            for mode in (0, 1):
                self._cpu.call("kush_cpu_write", self.D, self.bits, k.data_ptr(), v.data_ptr(), k.stride(0),
                               v.stride(0), query_start_loc.data_ptr(), seq_lens.data_ptr(), job_seq.data_ptr(),
                               job_page.data_ptr(), n_jobs, mode, cache.data_ptr(), bs, hs, tail_k.data_ptr(),
                               tail_idx.data_ptr(), block_table.data_ptr(), block_table.stride(0), H)
            return
        for mode in ((2,) if fused else (0, 1)):
            self._lib.call("kush_write_ex", self.D, self.bits, self._dt, k.data_ptr(), v.data_ptr(), k.stride(0),
                           v.stride(0), query_start_loc.data_ptr(), seq_lens.data_ptr(), tail_idx.data_ptr(),
                           job_seq.data_ptr(), job_page.data_ptr(), n_jobs, mode, cache.data_ptr(), bs, hs,
                           tail_k.data_ptr(), block_table.data_ptr(), block_table.stride(0), H, self._stream(),
                           int(bool(rot)))

    # ---------------------------------------------------------------- rotation
    def fwht(self, x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """Walsh-Hadamard rotation of every D-row of contiguous x in the canonical order (butterflies at
        strides 1..D/2, then fp32 1/sqrt(D)), bit-identical to the reference's CPU and GPU kernels
        (_ops.py:104-126); out (contiguous, x's shape and dtype) may be x. H @ H = I, so it also
        rotates back. Same rotation as rotate(x, hadamard(D)) up to fp32 rounding."""
        D = self.D
        _require(x.shape[-1] == D and x.is_contiguous(), f"fwht: x needs {D} contiguous elements per row")
        _require(x.dtype == self.dtype, f"fwht: x is {x.dtype}; these kernels were built for {self.dtype}")
        out = torch.empty_like(x) if out is None else out
        _require(out.is_contiguous() and out.shape == x.shape and out.dtype == x.dtype,
                 "fwht: out must be a contiguous tensor of x's shape and dtype")
        self._on_device(x=x, out=out)
        rows = x.numel() // D
        if rows and not self.gpu:                                # in place on the host
            if out.data_ptr() != x.data_ptr():
                out.copy_(x)
            self._cpu.call("kush_cpu_fwht", D, out.data_ptr(), rows)
        elif rows:
            self._lib.call("kush_fwht", D, self._dt, x.data_ptr(), out.data_ptr(), D, D, rows, self._stream())
        return out

    # ---------------------------------------------------------------- unpack (prefill with history)
    def unpack(self, cache: torch.Tensor, page_blk: torch.Tensor, page_dst: torch.Tensor, tail_blk: torch.Tensor,
               tail_info: torch.Tensor, tail_k: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
               new_dst: torch.Tensor, kp: torch.Tensor, vp: torch.Tensor, rot: bool) -> None:
        """One packed-prefill group's keys / values into kp, vp ([rows, Hkv, D], contiguous), one launch
        (_ops.py:128-180): full history pages (block page_blk[i] -> rows page_dst[i] + 0..31), partial pages
        (block tail_blk[i], tail_info[i] = (first row, tokens, tail slot): K from tail_k, V from the record)
        and the new chunk (row j of k_new / v_new [n, Hkv, D] -> row new_dst[j]). int32 index tensors. rot:
        rotate history back (canonical Walsh-Hadamard); new rows are copied as they are. Dequantization:
        fma(code, scale, bias) in fp32, rounded once to kp's dtype. Rows no entry names stay untouched."""
        H, D = kp.shape[1] if kp.dim() == 3 else -1, self.D
        n_pages, n_tail, n_new = page_blk.numel(), tail_blk.numel(), new_dst.numel()
        index = (page_blk, page_dst, tail_blk, tail_info, new_dst)
        _require(all(t.dtype == torch.int32 and t.is_contiguous() for t in index),
                 "unpack: page_blk, page_dst, tail_blk, tail_info and new_dst must be contiguous int32")
        _require(kp.dim() == 3 and kp.shape[2] == D and vp.shape == kp.shape and kp.is_contiguous()
                 and vp.is_contiguous(), f"unpack: kp and vp must be contiguous [rows, Hkv, {D}] of one shape")
        _require(all(t.dim() == 3 and t.shape[1:] == (H, D) and t.stride(2) == 1 and t.stride(1) == D
                     for t in (k_new, v_new)),
                 f"unpack: k_new and v_new must be [n, {H}, {D}] rows (unit dim stride, head stride {D})")
        _require(page_dst.numel() == n_pages, "unpack: page_dst needs one destination row per page_blk entry")
        _require(tail_info.numel() == 3 * n_tail, "unpack: tail_info needs (first row, tokens, slot) per tail_blk entry")
        _require(k_new.shape[0] >= n_new and v_new.shape[0] >= n_new, "unpack: k_new and v_new need a row per new_dst entry")
        for t in (tail_k, k_new, v_new, kp, vp):
            _require(t.dtype == self.dtype, f"unpack: tail_k, k_new, v_new, kp and vp must be {self.dtype}, got {t.dtype}")
        bs, hs = _byte_strides(cache)
        _require(cache.dim() >= 2 and cache.shape[1] >= H, "cache must be [blocks, >= Hkv, ...]")
        _require((cache.data_ptr() | bs | hs) % 16 == 0,
                 "cache records must start 16-byte aligned (pointer, block and head strides)")
        _require(tail_k.dim() == 4 and tail_k.shape[1:] == (H, PAGE, D) and tail_k.is_contiguous(),
                 f"tail_k must be contiguous [slots, {H}, {PAGE}, {D}]")
        self._on_device(cache=cache, page_blk=page_blk, page_dst=page_dst, tail_blk=tail_blk, tail_info=tail_info,
                        tail_k=tail_k, k_new=k_new, v_new=v_new, new_dst=new_dst, kp=kp, vp=vp)
        if n_pages + n_tail + n_new == 0:
            return
        if self._validating():
            check_unpack_indices(page_blk, page_dst, tail_blk, tail_info, new_dst, kp.shape[0], cache.shape[0],
                                 tail_k.shape[0])
        if not self.gpu:
            self._cpu.call("kush_cpu_unpack", D, self.bits, cache.data_ptr(), bs, hs, H, page_blk.data_ptr(),
                           page_dst.data_ptr(), n_pages, tail_blk.data_ptr(), tail_info.data_ptr(), n_tail,
                           tail_k.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), v_new.stride(0),
                           new_dst.data_ptr(), n_new, kp.data_ptr(), vp.data_ptr(), int(bool(rot)))
            return
        self._lib.call("kush_unpack", D, self.bits, self._dt, cache.data_ptr(), bs, hs, H, page_blk.data_ptr(),
                       page_dst.data_ptr(), n_pages, tail_blk.data_ptr(), tail_info.data_ptr(), n_tail,
                       tail_k.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), v_new.stride(0),
                       new_dst.data_ptr(), n_new, kp.data_ptr(), vp.data_ptr(), int(bool(rot)), self._stream())

    # ---------------------------------------------------------------- decode
    def splits(self, num_seqs: int, num_kv_heads: int, max_full_pages: int) -> int:
        """Split-K factor for MI355X: a power of two, doubled while the grid holds fewer workgroups
        than CUs (a decode workgroup holds a whole CU's page ring) and every split keeps >= 2 pages per
        wave; at most 256. As in the reference (_ops.py:182-189) the grid stays small, so a work
        buffer of CUs * G * (D + 2) floats per (sequence, kv head) pair always suffices."""
        ns = 1
        if not self.gpu:                                         # the host decode takes no splits (1 on CPU)
            return ns
        while (ns < 256 and num_seqs * num_kv_heads * ns < self.sms
               and max_full_pages // (2 * ns) >= 2 * DECODE_WAVES):
            ns *= 2
        return ns

    def waves(self, num_seqs: int, num_kv_heads: int, n_splits: int, max_pages: int | None = None) -> int:
        """Waves per decode workgroup (measured on MI355X): 4 for split counts of 8 and more that 4
        divides -- where the workgroups (a quarter of the splits per sequence, kv head and 16-head
        chunk) still fill the CUs the library then gives every wave a split of its own (C4 at NS 64 /
        128 / 256: 226 / 234 / 242 us against 243 / 271 / 332 at the best of 2 and 4 waves without),
        and below that the waves share each split (C4 at NS 8: 224.6 us against 254.8 at 2 waves);
        else 2 when the grid holds at least two workgroups per CU (smaller workgroups overlap one's
        start and merge with another's page loop; C3 213.7 against 220.1 at 4); else 4, one wave per
        SIMD (C2 33.0 us against 33.5 with 8 waves, C4 217.8 against 221.0: the second wave of a SIMD
        adds issue slots but no bandwidth, and with a static page assignment it finishes ~6 us after
        the first). max_pages is accepted for callers that pass it. A configuration whose ring does
        not fit in LDS runs fewer (the library picks)."""
        if n_splits >= 2 * DECODE_WAVES and n_splits % DECODE_WAVES == 0:
            return DECODE_WAVES                # wave splits where the grid allows (kush_decode.hip)
        if num_seqs * num_kv_heads * n_splits >= 2 * self.sms:
            return 2
        return DECODE_WAVES

    def decode(self, q: torch.Tensor, out: torch.Tensor, cache: torch.Tensor, block_table: torch.Tensor,
               seq_lens: torch.Tensor, tail_idx: torch.Tensor, tail_k: torch.Tensor,
               scale: float, n_splits: int = 1, work: torch.Tensor | None = None, *,
               waves: int | None = None, order: torch.Tensor | None = None, rot: bool = False) -> None:
        """out[s] = attention of q[s] ([Hq, D]) over the seq_lens[s] cached tokens of sequence s.
        n_splits > 1 needs `work` (fp32, >= S*Hkv*n_splits*G*(D+2) elements) (_ops.py:191-213); the
        splits are merged inside the same launch (split-K counters of this Ops), or by a second
        kernel when the batch exceeds the counters. waves: 2, 4 or 8 waves per workgroup (None:
        the waves() policy). order: optional int32 [S] permutation of the sequences, the order in
        which their workgroups start (longest first balances a ragged batch, e.g. from the host-side
        lengths a serving engine's metadata builder holds); it does not change the results. Calls on
        one Ops must not run concurrently on different streams (they share the counters, as the
        reference's callers share `work`). rot: the cache was written with rot=True: q is rotated on
        load and the output rotated back inside the kernels (no reference counterpart)."""
        self._decode(q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits, work, waves, order, rot,
                     None, None)

    def append_decode(self, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor, out: torch.Tensor,
                      cache: torch.Tensor, block_table: torch.Tensor, seq_lens: torch.Tensor, tail_idx: torch.Tensor,
                      tail_k: torch.Tensor, scale: float, n_splits: int = 1, work: torch.Tensor | None = None, *,
                      waves: int | None = None, order: torch.Tensor | None = None, rot: bool = False) -> None:
        """append(k, v, ..., pos_offset=-1, advance=False) followed by decode(q, out, ...), in one launch
        when it applies (at most 16 q heads per kv head, 16-byte aligned k / v rows; otherwise the two
        calls): row s of k / v is the token at position seq_lens[s] - 1, which seq_lens already counts
        (the serving engines' convention). The same bytes and outputs as the two calls. No reference
        counterpart."""
        S, H = q.shape[0], tail_k.shape[1]
        self._check_rows("k", k, H)
        self._check_rows("v", v, H)
        if k.shape[0] < S or v.shape[0] < S:
            raise ValueError("k and v need one row per sequence")
        e = k.element_size()
        aligned = ((k.data_ptr() | v.data_ptr() | (k.stride(0) * e) | (v.stride(0) * e)) & 15) == 0
        if self.G > 16 or not aligned or not self.gpu:
            self.append(k, v, seq_lens, tail_idx, cache, block_table, tail_k, -1, False, rot=rot)
            self.decode(q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits, work, waves=waves,
                        order=order, rot=rot)
            return
        self._on_device(k=k, v=v)
        self._decode(q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits, work, waves, order, rot,
                     k, v)

    def _decode(self, q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits, work, waves, order, rot,
                app_k, app_v) -> None:
        S, H = q.shape[0], tail_k.shape[1]
        G, D = self.G, self.D
        if q.shape != (S, H * G, D) or not q.is_contiguous() or q.dtype != self.dtype:
            raise ValueError(f"q must be contiguous {self.dtype} [S, {H * G}, {D}]")
        if out.shape != q.shape or not out.is_contiguous() or out.dtype != self.dtype:
            raise ValueError("out must be contiguous, with q's shape and dtype")
        self._check_index(seq_lens=seq_lens, tail_idx=tail_idx)
        self._check_cache(cache, block_table, tail_k, H)
        self._on_device(q=q, out=out, cache=cache, block_table=block_table, seq_lens=seq_lens, tail_idx=tail_idx,
                        tail_k=tail_k)
        if seq_lens.numel() < S or tail_idx.numel() < S or block_table.shape[0] < S:
            raise ValueError("seq_lens, tail_idx and block_table need one entry per sequence")
        if n_splits < 1:
            raise ValueError("n_splits must be >= 1")
        self._check_values(cache, block_table, seq_lens, tail_idx, tail_k, S)
        if not self.gpu:                # one pass per (sequence, kv head): splits, work, waves, order unused
            _require(not rot, "decode(rot=True) is a GPU extension; the CPU path takes a rotated q (fwht)")
            bs, hs = _byte_strides(cache)
            self._cpu.call("kush_cpu_decode", D, self.bits, q.data_ptr(), out.data_ptr(), cache.data_ptr(), bs, hs,
                           tail_k.data_ptr(), tail_idx.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(),
                           block_table.stride(0), H, G, float(scale), S)
            return
        part_ml = part_o = None
        if n_splits > 1:
            nml = S * H * n_splits * G * 2
            if (work is None or work.dtype != torch.float32 or not work.is_contiguous()
                    or work.numel() < nml + S * H * n_splits * G * D or work.device != self.device):
                raise ValueError(f"n_splits > 1 needs a contiguous fp32 work tensor of >= "
                                 f"{nml + S * H * n_splits * G * D} elements on {self.device}")
            part_ml, part_o = work.data_ptr(), work.data_ptr() + nml * 4
        if order is not None:
            self._check_index(order=order)
            self._on_device(order=order)
            if order.numel() < S:
                raise ValueError("order needs one entry per sequence")
            if self._validating() and not torch.equal(order[:S].sort().values.cpu(), torch.arange(S, dtype=torch.int32)):
                raise ValueError("order must be a permutation of the sequences")
        bs, hs = _byte_strides(cache)
        stream = self._stream()
        fused = n_splits > 1 and S * H * (-(-G // 16)) <= SYNC_SLOTS
        sync = self._sync.data_ptr() if fused else None
        wv = self.waves(S, H, n_splits, block_table.shape[1]) if waves is None else int(waves)
        ref = (D, self.bits, G, self._dt, q.data_ptr(), out.data_ptr(), cache.data_ptr(), bs, hs, tail_k.data_ptr(),
               tail_idx.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(), block_table.stride(0), H, float(scale),
               int(n_splits), part_ml, part_o, S, stream)
        ext = (min(block_table.shape[1], 1 << 30), sync, wv, order.data_ptr() if order is not None else None,
               int(bool(rot)))
        if app_k is None:
            self._lib.call("kush_decode_ex", *ref, *ext)
        else:
            self._lib.call("kush_append_decode", *ref, app_k.data_ptr(), app_v.data_ptr(), app_k.stride(0),
                           app_v.stride(0), *ext)
        if n_splits > 1 and not fused:
            self._lib.call("kush_combine_ex", D, G, self._dt, out.data_ptr(), part_ml, part_o, int(n_splits), H, S,
                           stream, int(bool(rot)))


# ---------------------------------------------------------------- page bookkeeping
def pages_touched(ctx: int, total: int) -> range:
    """Logical pages that receive tokens when positions [ctx, total) are added: from the page holding
    position ctx through the one holding total - 1 (_ops.py:342-344)."""
    if total <= ctx:
        return range(0)
    return range(ctx // PAGE, (total - 1) // PAGE + 1)


def _check_covers(query_start_loc: torch.Tensor, seq_lens: torch.Tensor, job_seq: torch.Tensor,
                  job_page: torch.Tensor) -> None:
    """A one-launch write (mode 2) needs a job for every page each sequence's new rows touch
    (pages_touched(seq_lens[s] - rows, seq_lens[s])): the first touched page's job reads a partly
    filled tail and the last one's writes the new tail. Raises ValueError naming the first sequence
    whose list misses a touched page."""
    qsl = query_start_loc.long().cpu().tolist()
    sl = seq_lens.long().cpu().tolist()
    have: dict[int, set] = {}
    for s_, p_ in zip(job_seq.long().cpu().tolist(), job_page.long().cpu().tolist()):
        have.setdefault(s_, set()).add(p_)
    for s_ in range(len(sl)):
        rows = qsl[s_ + 1] - qsl[s_]
        missing = [p_ for p_ in pages_touched(sl[s_] - rows, sl[s_]) if p_ not in have.get(s_, ())]
        if missing:
            raise ValueError(f"write(fused=True): the jobs of sequence {s_} miss touched page(s) {missing[:4]}; "
                             "list every page pages_touched gives, or write with fused=False (two launches)")


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


# The reference's _ops module also holds its torch helpers; they live in their own modules here and
# keep their reference names on this one.
from ._attention import attn_lse, history_attention, merge  # noqa: E402
from ._records import as_records, cached_kv, dequant_records  # noqa: E402
from ._rotation import FWHT_SCALE_BITS, fwht_reference, hadamard, rotate, rotation_enabled  # noqa: E402
