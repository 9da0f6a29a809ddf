"""CPU oracle bindings — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

ctypes bindings for ``oracle/libkush_oracle.so`` (a C restatement of the reference's CPU path,
kushkash/kush/cpu.mojo) and ``OracleOps``, an object with the method set of the reference's CPU
``Ops`` (kushkash/_ops.py:42-213, CPU branches). Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py use it, as the checker; the kushkash_amd package never imports it.

Every tensor handed to OracleOps must be fp32 on the CPU (the reference converts before its CPU
kernels: kushkash/cache.py:78), index tensors int32.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from functools import lru_cache
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB = HERE / "libkush_oracle.so"
PAGE = 32

_I, _F = ctypes.c_int64, ctypes.c_float
_SIGS = {   # argument lists of the reference's CPU C ABI (kushkash/_cpu.py:10-25)
    "kush_cpu_append": [_I] * 18,
    "kush_cpu_write": [_I] * 20,
    "kush_cpu_decode": [_I] * 14 + [_F, _I],
    "kush_cpu_fwht": [_I] * 3,
    "kush_cpu_unpack": [_I] * 22,
    "kush_oracle_set_threads": [_I],
    "kush_oracle_max_threads": [],
}


def build(force: bool = False) -> Path:
    """Compile the oracle with its Makefile (gcc); returns the library path. force: compile even when
    the library is newer than its source (make -B)."""
    if force or not LIB.exists() or LIB.stat().st_mtime < (HERE / "kush_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-B"] if force else ["make", "-s"], check=True, cwd=str(HERE))
    return LIB


@lru_cache(None)
def lib() -> ctypes.CDLL:
    if not LIB.exists():
        build()
    cdll = ctypes.CDLL(str(LIB))
    for name, args in _SIGS.items():
        fn = getattr(cdll, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int32
    return cdll


def call(name: str, *args) -> None:
    """Same error convention as the reference (kushkash/_cpu.py:38-40)."""
    if getattr(lib(), name)(*args) != 0:
        raise ValueError(f"{name}: unsupported head_dim/bits (CPU supports head_dim 64/128/256, bits 4/8)")


def set_threads(n: int) -> None:
    """Threads for decode (0 = all); the reference runs one task per (sequence, kv head)."""
    lib().kush_oracle_set_threads(int(n))


def max_threads() -> int:
    return int(lib().kush_oracle_max_threads())


def _byte_strides(cache: torch.Tensor) -> tuple[int, int]:
    e = cache.element_size()
    return cache.stride(0) * e, cache.stride(1) * e


class OracleOps:
    """The reference's CPU ``Ops`` surface (kushkash/_ops.py:42-213) over the C restatement."""

    def __init__(self, device, head_dim: int, bits: int, group: int, dtype: torch.dtype = torch.float32):
        self.device = torch.device(device)
        if self.device.type != "cpu":
            raise ValueError("OracleOps runs on the CPU only")
        if head_dim not in (64, 128, 256):
            raise ValueError("CPU head_dim must be 64, 128 or 256")
        self.D, self.bits, self.G, self.dtype = head_dim, bits, group, dtype
        self.gpu = False
        self.sms = 1

    def append(self, k, v, seq_lens, tail_idx, cache, block_table, tail_k, pos_offset: int, advance: bool) -> None:
        S, H = k.shape[0], k.shape[1]
        bs, hs = _byte_strides(cache)
        call("kush_cpu_append", self.D, self.bits, k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0),
             seq_lens.data_ptr(), pos_offset, int(advance), cache.data_ptr(), bs, hs, tail_k.data_ptr(),
             tail_idx.data_ptr(), block_table.data_ptr(), block_table.stride(0), H, S)

    def write(self, k, v, query_start_loc, seq_lens, tail_idx, job_seq, job_page, cache, block_table, tail_k, *,
              fused: bool = False) -> None:
        """The reference's two ordered modes (0, then 1); `fused` (Ops.write's one-launch declaration) is
        accepted and changes nothing here: for a complete job list both give the same bytes."""
        n_jobs, H = job_seq.numel(), k.shape[1]
        if n_jobs == 0:
            return
        bs, hs = _byte_strides(cache)
        for mode in (0, 1):
            call("kush_cpu_write", self.D, self.bits, k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0),
                 query_start_loc.data_ptr(), seq_lens.data_ptr(), job_seq.data_ptr(), job_page.data_ptr(), n_jobs,
                 mode, cache.data_ptr(), bs, hs, tail_k.data_ptr(), tail_idx.data_ptr(), block_table.data_ptr(),
                 block_table.stride(0), H)

    def fwht(self, x, out=None):
        D = self.D
        if x.shape[-1] != D or not x.is_contiguous() or x.dtype != torch.float32:
            raise ValueError(f"fwht: x must be contiguous fp32 with last dim {D}")
        out = torch.empty_like(x) if out is None else out
        if out.data_ptr() != x.data_ptr():
            out.copy_(x)
        rows = x.numel() // D
        if rows:
            call("kush_cpu_fwht", D, out.data_ptr(), rows)
        return out

    def unpack(self, cache, page_blk, page_dst, tail_blk, tail_info, tail_k, k_new, v_new, new_dst, kp, vp,
               rot: bool) -> None:
        H = kp.shape[1]
        n_pages, n_tail, n_new = page_blk.numel(), tail_blk.numel(), new_dst.numel()
        if n_pages + n_tail + n_new == 0:
            return
        bs, hs = _byte_strides(cache)
        call("kush_cpu_unpack", self.D, self.bits, cache.data_ptr(), bs, hs, H, page_blk.data_ptr(),
             page_dst.data_ptr(), n_pages, tail_blk.data_ptr(), tail_info.data_ptr(), n_tail, tail_k.data_ptr(),
             k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), v_new.stride(0), new_dst.data_ptr(), n_new,
             kp.data_ptr(), vp.data_ptr(), int(rot))

    def splits(self, num_seqs: int, num_kv_heads: int, max_full_pages: int) -> int:
        return 1

    def decode(self, q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale: float, n_splits: int = 1,
               work=None) -> None:
        S, H = q.shape[0], tail_k.shape[1]
        bs, hs = _byte_strides(cache)
        call("kush_cpu_decode", self.D, self.bits, q.data_ptr(), out.data_ptr(), cache.data_ptr(), bs, hs,
             tail_k.data_ptr(), tail_idx.data_ptr(), block_table.data_ptr(), seq_lens.data_ptr(),
             block_table.stride(0), H, self.G, float(scale), S)

    def append_decode(self, k, v, q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale: float,
                      n_splits: int = 1, work=None, **kw) -> None:
        """The reference's two calls in order: append at seq_lens - 1 (already counted), then decode."""
        self.append(k, v, seq_lens, tail_idx, cache, block_table, tail_k, pos_offset=-1, advance=False)
        self.decode(q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits, work)


if os.environ.get("KUSH_ORACLE_THREADS"):
    set_threads(int(os.environ["KUSH_ORACLE_THREADS"]))
