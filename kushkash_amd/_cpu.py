"""ctypes binding of the CPU path's host library (kushkash_amd/libkushcpu.so, csrc/kush_cpu.cpp): the
page-record kernels on the host, for Ops and KushCache on device "cpu". Its entry points keep the C ABI
of the reference's CPU library (kushkash/_cpu.py:10-25): every argument an int64 except the decode's
softmax scale. Missing library -> the first call raises, naming the build command.
"""
from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

LIB = Path(__file__).resolve().parent / "libkushcpu.so"

# Each entry point's parameters by name, in order, as include/kushkash_amd_cpu.h declares them: int64
# (an address, stride or count) except the float softmax scale.
PARAMS = {
    "kush_cpu_append": "head_dim bits k v k_row_stride v_row_stride seq_lens pos_offset advance cache "
                       "block_stride head_stride tail_k tail_idx block_table bt_row_stride hkv n_seqs",
    "kush_cpu_write": "head_dim bits k v k_row_stride v_row_stride query_start_loc seq_lens job_seq job_page "
                      "n_jobs mode cache block_stride head_stride tail_k tail_idx block_table bt_row_stride hkv",
    "kush_cpu_decode": "head_dim bits q out cache block_stride head_stride tail_k tail_idx block_table seq_lens "
                       "bt_row_stride hkv group scale n_seqs",
    "kush_cpu_fwht": "head_dim x rows",
    "kush_cpu_unpack": "head_dim bits cache block_stride head_stride hkv page_blk page_dst n_pages tail_blk "
                       "tail_info n_tail tail_k k_new v_new k_row_stride v_row_stride new_dst n_new kp vp rot",
    "kush_cpu_half_bits": "x out n",          # fp32 -> fp16 bits with the library's rounding (tests)
}
SIGNATURES = {name: [ctypes.c_float if p == "scale" else ctypes.c_int64 for p in params.split()]
              for name, params in PARAMS.items()}


@lru_cache(None)
def lib() -> ctypes.CDLL:
    if not LIB.exists():
        raise RuntimeError(f"kushkash_amd: {LIB.name} is not built; run `python -m kushkash_amd.build`")
    cdll = ctypes.CDLL(str(LIB))
    for name, args in SIGNATURES.items():
        fn = getattr(cdll, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int32
    return cdll


def call(name: str, *args) -> None:
    """Run one entry point; -1 (unsupported head_dim / bits) -> ValueError, as the reference's CPU path
    (kushkash/_cpu.py:38-40)."""
    if getattr(lib(), name)(*args) != 0:
        raise ValueError(f"{name}: unsupported head_dim/bits (CPU supports head_dim 64/128/256, bits 4/8)")
