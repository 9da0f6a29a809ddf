"""The timeline build (kushkash_amd/libkushhip_timeline.so, read by bench.py --timeline) runs the same
decode as the product library: bit-identical outputs on one input, and its records hold, per
workgroup, phases in time order, an XCD id in 0..7 and every wave's pages-done time between the
workgroup's start and its output (needs an MI355X)."""
import ctypes
import importlib
import math

import numpy as np
import pytest
import torch

import bench
from kushkash_amd import _lib

pytestmark = pytest.mark.gpu
kbuild = importlib.import_module("kushkash_amd.build")


@pytest.mark.parametrize("waves", [4, 8])
def test_timeline_build_matches_the_product(waves):
    a = bench.parse_args(["--pools", "1", "--batch", "8", "--ctx", "1000"])   # 31 full pages + a 8-token tail
    w = bench.make_workload(a, "cuda:0")
    ops, B, Hkv, G, D = w["ops"], w["B"], w["Hkv"], w["G"], w["D"]
    work = torch.empty(B * Hkv * G * (D + 2), dtype=torch.float32, device="cuda:0")

    def run():
        out = torch.empty_like(w["q"])
        ops.decode(w["q"], out, w["cache"], w["tables"][0], w["seq_lens"], w["tail_idx"], w["tail_k"],
                   1.0 / math.sqrt(D), 1, work, waves=waves)
        torch.cuda.synchronize()
        return out

    product = run()
    assert _lib.LIB != kbuild.TIMELINE_LIB
    saved = _lib.LIB
    try:
        _lib.LIB = kbuild.TIMELINE_LIB
        _lib.lib.cache_clear()
        timed = run()
        read = _lib.lib().kush_timeline_read
        read.argtypes, read.restype = [ctypes.c_void_p, ctypes.c_int64], ctypes.c_int32
        rows = B * Hkv
        buf = np.zeros((rows, 16), dtype=np.int64)
        assert read(buf.ctypes.data_as(ctypes.c_void_p), rows) == 0
    finally:
        _lib.LIB = saved
        _lib.lib.cache_clear()
    assert torch.equal(product, timed)
    wall = buf[:, :5]
    assert (wall > 0).all()
    assert (np.diff(wall, axis=1) >= 0).all(), "phases out of order"
    assert (buf[:, 6] >= buf[:, 5]).all()
    assert ((buf[:, 7] >= 0) & (buf[:, 7] < 8)).all()
    waves_done = buf[:, 8:8 + waves]
    assert (waves_done >= wall[:, :1]).all() and (waves_done <= wall[:, 4:5]).all()
    assert (wall[:, 4] - wall[:, 0] < 100 * 10_000).all()      # each workgroup within 10 ms (100 MHz clock)
