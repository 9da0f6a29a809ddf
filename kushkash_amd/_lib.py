"""ctypes binding of the gfx950 HIP library over its C ABI (include/kushkash_amd.h).

Replaces the reference's two launch backends (kushkash/_cuda.py: PTX through the CUDA driver API;
kushkash/_cpu.py: the Mojo CPU library): every kernel here is a plain C function taking device
pointers, sizes and a hipStream_t. There is no fallback: if the library is missing the first call
raises, naming the build command.
"""
from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

import torch   # noqa: F401  -- loads torch's HIP runtime first; the library binds to it (same soname)

LIB = Path(__file__).resolve().parent / "libkushhip.so"
ABI_VERSION = 8

_P, _I32, _I64, _F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float

# head_dim, bits, dtype, k, v, k_row_stride, v_row_stride, seq_lens, pos_offset, advance, tail_idx, cache,
# block_stride, head_stride, tail_k, block_table, bt_row_stride, hkv, n_seqs, stream
_APPEND = [_I32, _I32, _I32, _P, _P, _I64, _I64, _P, _I32, _I32, _P, _P, _I64, _I64, _P, _P, _I64, _I32, _I32, _P]
# head_dim, bits, dtype, k, v, k_row_stride, v_row_stride, query_start_loc, seq_lens, tail_idx, job_seq, job_page,
# n_jobs, mode, cache, block_stride, head_stride, tail_k, block_table, bt_row_stride, hkv, stream
_WRITE = [_I32, _I32, _I32, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _I32, _I32, _P, _I64, _I64, _P, _P, _I64, _I32, _P]
# head_dim, bits, group, dtype, q, out, cache, block_stride, head_stride, tail_k, tail_idx, block_table, seq_lens,
# bt_row_stride, hkv, scale, n_splits, part_ml, part_o, n_seqs, stream
_DECODE = [_I32, _I32, _I32, _I32, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _I64, _I32, _F, _I32, _P, _P, _I32, _P]
# bt_cols, split_sync, waves, seq_order, rot
_DECODE_EXT = [_I32, _P, _I32, _P, _I32]
# head_dim, group, dtype, out, part_ml, part_o, n_splits, hkv, n_seqs, stream
_COMBINE = [_I32, _I32, _I32, _P, _P, _P, _I32, _I32, _I32, _P]

# Each reference entry point takes the reference's argument list; its `_ex` variant appends this
# library's extensions after the stream (include/kushkash_amd.h).
SIGNATURES = {
    "kush_append": _APPEND,
    "kush_append_ex": _APPEND + [_I32],                          # + rot
    "kush_write": _WRITE,
    "kush_write_ex": _WRITE + [_I32],                            # + rot
    "kush_decode": _DECODE,
    "kush_decode_ex": _DECODE + _DECODE_EXT,
    # + k, v, k_row_stride, v_row_stride, then the decode extensions
    "kush_append_decode": _DECODE + [_P, _P, _I64, _I64] + _DECODE_EXT,
    # the decode list without part_ml / part_o, then bt_cols, waves, seq_order, rot (no split_sync)
    "kush_decode_noalloc": _DECODE[:17] + [_I32, _P, _I32, _I32, _P, _I32],
    "kush_combine": _COMBINE,
    "kush_combine_ex": _COMBINE + [_I32],                        # + rot
    # head_dim, dtype, x, y, x_row_stride, y_row_stride, rows, stream
    "kush_fwht": [_I32, _I32, _P, _P, _I64, _I64, _I64, _P],
    # head_dim, bits, dtype, cache, block_stride, head_stride, hkv, page_blk, page_dst, n_pages, tail_blk, tail_info,
    # n_tail, tail_k, k_new, v_new, k_stride, v_stride, new_dst, n_new, kp, vp, rot, stream
    "kush_unpack": [_I32, _I32, _I32, _P, _I64, _I64, _I32, _P, _P, _I64, _P, _P, _I64, _P, _P, _P, _I64, _I64, _P,
                    _I64, _P, _P, _I32, _P],
    "kush_last_error": [],
    "kush_abi_version": [],
}


@lru_cache(None)
def lib() -> ctypes.CDLL:
    if not LIB.exists():
        raise RuntimeError(f"kushkash_amd: {LIB.name} is not built; run `python -m kushkash_amd.build` "
                           "(hipcc, gfx950)")
    cdll = ctypes.CDLL(str(LIB))
    for name, args in SIGNATURES.items():
        fn = getattr(cdll, name)
        fn.argtypes = args
        fn.restype = ctypes.c_char_p if name == "kush_last_error" else ctypes.c_int32
    if cdll.kush_abi_version() != ABI_VERSION:
        raise RuntimeError(f"kushkash_amd: {LIB.name} has ABI {cdll.kush_abi_version()}, expected {ABI_VERSION}; "
                           "rebuild it")
    return cdll


def call(name: str, *args) -> None:
    """Run one entry point; -1 (unsupported shape) -> ValueError like the reference's CPU path
    (kushkash/_cpu.py:38-40), any other failure -> RuntimeError with the library's message."""
    rc = getattr(lib(), name)(*args)
    if rc == 0:
        return
    msg = (lib().kush_last_error() or b"").decode(errors="replace")
    if rc == -1:
        raise ValueError(msg)
    raise RuntimeError(f"{name} failed ({rc}): {msg}")
