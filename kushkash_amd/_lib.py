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
ABI_VERSION = 7

_P, _I32, _I64, _F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
SIGNATURES = {
    # head_dim, bits, dtype, k, v, k_row_stride, v_row_stride, seq_lens, pos_offset, advance, tail_idx,
    # cache, block_stride, head_stride, tail_k, block_table, bt_row_stride, hkv, n_seqs, rot, stream
    "kush_append": [_I32, _I32, _I32, _P, _P, _I64, _I64, _P, _I32, _I32, _P, _P, _I64, _I64, _P, _P, _I64, _I32,
                    _I32, _I32, _P],
    # head_dim, bits, dtype, k, v, k_row_stride, v_row_stride, query_start_loc, seq_lens, tail_idx, job_seq,
    # job_page, n_jobs, mode, cache, block_stride, head_stride, tail_k, block_table, bt_row_stride, hkv, rot, stream
    "kush_write": [_I32, _I32, _I32, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _I32, _I32, _P, _I64, _I64, _P, _P,
                   _I64, _I32, _I32, _P],
    # head_dim, bits, group, dtype, q, out, cache, block_stride, head_stride, tail_k, tail_idx, block_table,
    # seq_lens, bt_row_stride, bt_cols, hkv, scale, n_splits, part_ml, part_o, split_sync, waves, seq_order, n_seqs,
    # rot, stream
    "kush_decode": [_I32, _I32, _I32, _I32, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _I64, _I32, _I32, _F, _I32, _P,
                    _P, _P, _I32, _P, _I32, _I32, _P],
    # head_dim, bits, group, dtype, k, v, k_row_stride, v_row_stride, q, out, cache, block_stride, head_stride,
    # tail_k, tail_idx, block_table, seq_lens, bt_row_stride, bt_cols, hkv, scale, n_splits, part_ml, part_o,
    # split_sync, waves, seq_order, n_seqs, rot, stream
    "kush_append_decode": [_I32, _I32, _I32, _I32, _P, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _I64,
                           _I32, _I32, _F, _I32, _P, _P, _P, _I32, _P, _I32, _I32, _P],
    # head_dim, group, dtype, out, part_ml, part_o, n_splits, hkv, n_seqs, rot, stream
    "kush_combine": [_I32, _I32, _I32, _P, _P, _P, _I32, _I32, _I32, _I32, _P],
    # head_dim, dtype, x, y, x_row_stride, y_row_stride, rows, stream
    "kush_fwht": [_I32, _I32, _P, _P, _I64, _I64, _I64, _P],
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
