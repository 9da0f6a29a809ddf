"""The streaming-floor measurement library (kushkash_amd/libkushfloor.so, read by bench.py --floor)
reads every full page of the workload exactly once in each launch shape: the xor of its per-lane
sums (the first KB of every record, each dword once) is the same for the decode's grid (mode 0),
the page-range grid (mode 1) and the persistent dynamic-chunk grid (mode 2, chunks claimed from a
device counter), computed independently on the host from the cache bytes; in mode 2 the
workgroups' chunk counts add up to the chunk total, in launch after launch on one counter, with
partial last pages (needs an MI355X)."""
import numpy as np
import pytest
import torch

import bench
from kushkash_amd._ops import PAGE

pytestmark = pytest.mark.gpu


def _workload(ctx, batch=8):
    a = bench.parse_args(["--pools", "1", "--batch", str(batch), "--ctx", str(ctx)])
    return bench.make_workload(a, "cuda:0")


def _expected_xor(w):
    """xor over every full page of every (sequence, kv head) of the dwords in its record's first KB."""
    cache, table = w["cache"].cpu().numpy(), w["tables"][0].cpu().numpy()
    full = int(w["seq_lens"][0].item()) // PAGE
    acc = np.uint32(0)
    for s in range(w["B"]):
        for p in range(full):
            rec = cache[table[s, p], :, :1024]                       # [Hkv, 1024] bytes
            acc ^= np.bitwise_xor.reduce(np.ascontiguousarray(rec).view(np.uint32).reshape(-1))
    return acc


def _xor(sums):
    return np.bitwise_xor.reduce(sums.cpu().numpy().view(np.uint32).reshape(-1))


@pytest.mark.parametrize("ctx", [4096, 1000, 100])
def test_every_page_once_in_every_launch_shape(ctx):
    w = _workload(ctx)
    want = _expected_xor(w)
    shapes = [(0, 4, 2, 1, 4), (0, 8, 2, 1, 4), (1, 4, 2, 3, 4), (2, 4, 2, 16, 4), (2, 4, 2, 8, 8), (2, 8, 2, 8, 4)]
    cp = lambda waves, pw: 2 * waves * pw
    for mode, waves, depth, z, pw in shapes:
        cps = -(-w["pages"] // cp(waves, pw))
        n_chunks = w["B"] * w["Hkv"] * cps
        if mode == 2 and (z > n_chunks or cps * cp(waves, pw) > w["pages"]):
            continue                 # mode 2 reads a whole chunk's ids: the table must hold them
        fl = bench.FloorLaunches(w, mode, waves, depth, z, pw, marks=True)    # one launch at construction
        for rep in range(3):
            torch.cuda.synchronize()
            assert _xor(fl.sums) == want, (mode, waves, depth, z, pw, rep)
            if mode == 2:
                chunks = fl.marks[:, 5].cpu().numpy()
                assert chunks.sum() == n_chunks and (chunks >= 1).all(), (chunks.sum(), n_chunks)
            fl.sums.zero_()
            fl.run(rep + 1, 1)
        torch.cuda.synchronize()
        assert _xor(fl.sums) == want
