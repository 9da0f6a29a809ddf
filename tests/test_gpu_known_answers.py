"""The HIP path against the known answers of tests/golden/known_answers.npz (needs an MI355X):
records written on the GPU from fp32 inputs are the constructed bytes, and decode over them matches
the float64 attention outputs within the decode tolerance."""
from pathlib import Path

import numpy as np
import pytest
import torch

import kushkash_amd as kk
from _harness import assert_out_close

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.npz"


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN) as z:
        return {k: z[k] for k in z.files}


def _gpu_cache(K, V, D, bits, G=1, appends=False):
    H, n = K.shape[0], K.shape[1]
    c = kk.KushCache(1, H, H * G, D, batch_size=1, bits=bits, device="cuda", dtype=torch.float32, rotate=False)
    k, v = torch.from_numpy(K)[None].cuda(), torch.from_numpy(V)[None].cuda()
    if appends and n > 40:
        c.write(0, k[:, :, :40], v[:, :, :40])
        for t in range(40, n):
            c.write(0, k[:, :, t:t + 1], v[:, :, t:t + 1])
    else:
        c.write(0, k, v)
    return c


def _records(c, pages):
    return np.stack([c.pool[0, int(c.block_table[0, p])].cpu().numpy() for p in range(pages)])


@pytest.mark.parametrize("appends", [False, True])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("D", [64, 128])
def test_gpu_exact_records_and_decode(golden, D, bits, appends):
    key = f"exact_D{D}_b{bits}_"
    G = int(golden[key + "G"])
    c = _gpu_cache(golden[key + "K"], golden[key + "V"], D, bits, G=G, appends=appends)
    want = golden[key + "rec"]
    got = _records(c, want.shape[0])
    assert np.array_equal(got, want), f"{(got != want).mean():.2e} of record bytes differ"
    c.scale = float(golden[key + "scale"])
    q = torch.from_numpy(golden[key + "q"])[None].cuda()
    for qq, ref in ((q, golden[key + "out"]), (torch.zeros_like(q), golden[key + "out_q0"])):
        out = c.attend(0, qq)[0].double().cpu().numpy()
        # max-abs 2e-3 at unit output scale; these constructed V reach |485|, where the bound is
        # relative: 2e-3 * max(1, max |ref|) (fp16 weights carry 2^-11 relative rounding)
        scale = max(1.0, float(np.abs(ref).max()))
        assert_out_close(torch.from_numpy(out), torch.from_numpy(ref), torch.float32, base=2e-3 * scale)


@pytest.mark.parametrize("case,bits", [("ties", 4), ("const", 4), ("const", 8), ("clamp", 4)])
def test_gpu_special_records(golden, case, bits):
    key = f"{case}_D64_b{bits}_"
    c = _gpu_cache(golden[key + "K"], golden[key + "V"], 64, bits)
    assert np.array_equal(_records(c, 1), golden[key + "rec"])
