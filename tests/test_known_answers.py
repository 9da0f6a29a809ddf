"""The CPU oracle against known answers (tests/golden/known_answers.npz, built by construction by
tests/golden/make_known_answers.py) and against a brute-force nearest-level search. These pin the
oracle independently of its own formulas: exact records for inputs whose scales, offsets and codes
are fixed by construction, round-half-to-even ties, constant groups (scale 0), the clamp at a
subnormal fp16 scale, and decode outputs that reduce to float64 softmax attention."""
from pathlib import Path

import numpy as np
import pytest
import torch

from _harness import oracle_cache, split_record
from kushkash_amd._ops import PAGE, record_bytes

GOLDEN = Path(__file__).resolve().parent / "golden" / "known_answers.npz"


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN) as z:          # plain arrays: no pickle
        return {k: z[k] for k in z.files}


def _cache_from(K: np.ndarray, V: np.ndarray, D: int, bits: int, G: int = 1, appends: bool = False):
    """Oracle-backed cache holding one sequence: K, V [H, n, D] written in bulk, or 40 tokens in bulk
    and the rest one token at a time."""
    H, n = K.shape[0], K.shape[1]
    c = oracle_cache(1, H, H * G, D, batch_size=1, bits=bits, rotate=False)
    k, v = torch.from_numpy(K)[None], torch.from_numpy(V)[None]
    if appends and n > 40:
        c.write(0, k[:, :, :40], v[:, :, :40])
        for t in range(40, n):
            c.write(0, k[:, :, t:t + 1], v[:, :, t:t + 1])
    else:
        c.write(0, k, v)
    return c


def _records(c, pages: int) -> np.ndarray:
    return np.stack([c.pool[0, int(c.block_table[0, p])].numpy() for p in range(pages)])


@pytest.mark.parametrize("appends", [False, True])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("D", [64, 128])
def test_exact_records(golden, D, bits, appends):
    """Inputs b + c s with fp16-exact dyadic s, b and codes reaching both extremes: the records are
    exactly the constructed bytes, by bulk write and by token appends."""
    key = f"exact_D{D}_b{bits}_"
    c = _cache_from(golden[key + "K"], golden[key + "V"], D, bits, appends=appends)
    want = golden[key + "rec"]
    assert want.shape[-1] == record_bytes(D, bits)
    got = _records(c, want.shape[0])
    assert np.array_equal(got, want), f"{(got != want).mean():.2e} of record bytes differ"


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("D", [64, 128])
def test_exact_decode(golden, D, bits):
    """Over exactly dequantizable records the decode output is softmax attention in float64 (q random),
    and the plain mean of V for q = 0."""
    key = f"exact_D{D}_b{bits}_"
    G = int(golden[key + "G"])
    c = _cache_from(golden[key + "K"], golden[key + "V"], D, bits, G=G)
    c.scale = float(golden[key + "scale"])
    q = torch.from_numpy(golden[key + "q"])[None]
    out = c.attend(0, q)[0].double().numpy()
    want = golden[key + "out"]
    assert np.abs(out - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    out0 = c.attend(0, torch.zeros_like(q))[0].double().numpy()
    assert np.abs(out0 - golden[key + "out_q0"]).max() <= 1e-5 * max(1.0, np.abs(golden[key + "out_q0"]).max())


@pytest.mark.parametrize("case,bits", [("ties", 4), ("const", 4), ("const", 8), ("clamp", 4)])
def test_special_records(golden, case, bits):
    """Round-half-to-even ties, constant channel / row (scale 0, code 0, offset fp16(value)) and the
    clamp at a subnormal fp16 scale."""
    key = f"{case}_D64_b{bits}_"
    c = _cache_from(golden[key + "K"], golden[key + "V"], 64, bits)
    want = golden[key + "rec"]
    got = _records(c, 1)
    if not np.array_equal(got, want):
        kq, ks, kb, vq, vs, vb = split_record(torch.from_numpy(got[0, 0]), 64, bits)
        wq, wks, wkb, wvq, wvs, wvb = split_record(torch.from_numpy(want[0, 0]), 64, bits)
        raise AssertionError(f"K codes differ at {(kq != wq).nonzero()[:5].tolist()}, V codes at "
                             f"{(vq != wvq).nonzero()[:5].tolist()}, ks {(ks != wks).sum()}, kb {(kb != wkb).sum()}, "
                             f"vs {(vs != wvs).sum()}, vb {(vb != wvb).sum()}")


def _nearest_level(y: torch.Tensor, half: int) -> torch.Tensor:
    """Brute force: the code in [-half, half - 1] nearest to y, ties to the even code."""
    cand = torch.arange(-half, half, dtype=torch.float64)
    d = (y.double()[..., None] - cand).abs()
    best = d.min(-1, keepdim=True).values
    hit = d == best
    even = cand.remainder(2) == 0
    pick = torch.where(hit.sum(-1, keepdim=True) > 1, hit & even, hit)
    return cand[pick.float().argmax(-1)].to(torch.int64)


@pytest.mark.parametrize("bits", [4, 8])
def test_codes_are_nearest_levels(bits):
    """Given the stored fp16 scale and offset, every code is the nearest level to x (brute force
    over all 2^bits levels, ties to even, out-of-range values clamped), for inputs spanning wide,
    tiny (fp16-subnormal scales) and mixed ranges."""
    torch.manual_seed(bits)
    D, H, half = 64, 3, 2 ** (bits - 1)
    K = torch.randn(1, H, PAGE, D) * torch.tensor([3.0, 1e-6, 40.0])[None, :, None, None]
    V = torch.randn(1, H, PAGE, D) * torch.tensor([1.0, 3e-7, 100.0])[None, :, None, None]
    K[0, 0, :, 7] += 1000.0
    c = oracle_cache(1, H, H, D, batch_size=1, bits=bits, rotate=False)
    c.write(0, K, V)
    kq, ks, kb, vq, vs, vb = split_record(c.pool[0, int(c.block_table[0, 0])], D, bits)
    for x, q, s, b in ((K[0], kq, ks[:, None, :], kb[:, None, :]), (V[0], vq, vs[..., None], vb[..., None])):
        inv = torch.where(s > 0, 1.0 / s, torch.zeros_like(s))             # fp32, as the format defines
        y = (x - b) * inv
        assert torch.equal(q.long(), _nearest_level(y, half))


def test_padding_rows_and_empty_sequences():
    """Append with pos_offset = -1 (vLLM positions): a row whose position is negative (an empty
    sequence) writes nothing; the others land at seq_len - 1 (reference: gpu.mojo:222-223)."""
    from oracle.cpu_ops import OracleOps
    D, bits, H = 64, 4, 2
    ops = OracleOps("cpu", D, bits, 1)
    S, pages = 3, 2
    cache = torch.zeros(S * pages, H, record_bytes(D, bits), dtype=torch.uint8)
    bt = torch.arange(S * pages, dtype=torch.int32).view(S, pages)
    tail_k = torch.full((S, H, PAGE, D), 7.0)
    tail_idx = torch.arange(S, dtype=torch.int32)
    lens = torch.tensor([0, 1, 32], dtype=torch.int32)          # row 0: position -1 (padding)
    k, v = torch.randn(S, H, D), torch.randn(S, H, D)
    before = cache.clone(), tail_k.clone()
    ops.append(k, v, lens, tail_idx, cache, bt, tail_k, pos_offset=-1, advance=False)
    assert torch.equal(lens, torch.tensor([0, 1, 32], dtype=torch.int32))
    assert torch.equal(cache[0:2], before[0][0:2]) and torch.equal(tail_k[0], before[1][0])
    assert torch.equal(tail_k[1, :, 0], k[1])                    # position 0 of sequence 1: K exact in the tail
    assert not torch.equal(cache[bt[2, 0]], before[0][bt[2, 0]])  # position 31 completed page 0 of sequence 2
