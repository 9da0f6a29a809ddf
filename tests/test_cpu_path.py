"""The package's CPU path (Ops / KushCache on device "cpu": the host library libkushcpu.so,
csrc/kush_cpu.cpp), checked the way the reference checks its CPU path (tests/test_cpu.py,
tests/test_ragged.py) and against the oracle on the same inputs: records and tails byte-identical,
decode within fp32 rounding of the oracle's and of float64 attention over the cached values, the
rotation and the unpack bit-identical, the fp16 rounding of scales and biases that of numpy."""
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import kushkash_amd
from _harness import oracle_cache, ref_quantize, split_record
from kushkash_amd import _cpu
from kushkash_amd._ops import PAGE, Ops, hadamard, record_bytes
from oracle.cpu_ops import OracleOps
from test_oracle import RaggedHost


def cpu_cache(*args, **kw) -> kushkash_amd.KushCache:
    return kushkash_amd.KushCache(*args, **dict(kw, device="cpu", dtype=torch.float32))


def test_cpu_ops_surface():
    ops = Ops(torch.device("cpu"), 128, 4, 7, torch.float32)
    assert not ops.gpu and ops.splits(64, 4, 128) == 1 and ops.cfg.arch == "cpu"
    with pytest.raises(ValueError, match="fp32"):
        Ops(torch.device("cpu"), 128, 4, 7, torch.bfloat16)
    with pytest.raises(ValueError, match="head_dim"):
        Ops(torch.device("cpu"), 96, 4, 7, torch.float32)
    with pytest.raises(ValueError, match="rotate_in_kernels"):
        cpu_cache(1, 2, 2, 64, rotate=True, rotate_in_kernels=True)


def test_half_rounding_matches_numpy():
    """fp32 -> fp16 of the library (the scales and biases of every record), round to nearest even,
    on 2^22 values spread over every exponent plus the edges: subnormal halves, the overflow
    threshold 65520, infinities and signed zeros."""
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                      2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1e-30, np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([bits.view(np.float32), edges])
    x = x[~np.isnan(x)]
    got = np.empty(x.size, dtype=np.uint16)
    assert _cpu.lib().kush_cpu_half_bits(x.ctypes.data, got.ctypes.data, x.size) == 0
    with np.errstate(over="ignore"):                      # past 65520: infinity, as the library
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want), x[got != want][:8]


@pytest.mark.parametrize("rot", [False, True])
@pytest.mark.parametrize("appends", [False, True])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("bits", [4, 8])
def test_records_and_tails_equal_the_oracle(bits, D, appends, rot):
    """Bulk writes and token appends through KushCache: the product's pool and tails byte-equal to the
    oracle's, and (unrotated) the reference test's codes and scales (tests/test_cpu.py:40-76)."""
    torch.manual_seed(D + bits + 7 * appends)
    B, H, T = 2, 3, 3 * PAGE + 5
    K, V = torch.randn(B, H, T, D) * 3, torch.randn(B, H, T, D)
    caches = [cpu_cache(1, H, H, D, batch_size=B, bits=bits, rotate=rot),
              oracle_cache(1, H, H, D, batch_size=B, bits=bits, rotate=rot)]
    for c in caches:
        if appends:
            c.write(0, K[:, :, :40], V[:, :, :40])
            for t in range(40, T):
                c.write(0, K[:, :, t:t + 1], V[:, :, t:t + 1])
        else:
            c.write(0, K, V)
    prod, orc = caches
    assert torch.equal(prod.pool, orc.pool) and torch.equal(prod.tail_k, orc.tail_k)
    if rot:
        return
    for b in range(B):
        for p in range(T // PAGE):
            kq, ks, kb, vq, vs, vb = split_record(prod.pool[0, int(prod.block_table[b, p])], D, bits)
            ck, sk, bk = ref_quantize(K[b, :, p * PAGE:(p + 1) * PAGE], bits, dim=1)
            cv, sv, bv = ref_quantize(V[b, :, p * PAGE:(p + 1) * PAGE], bits, dim=2)
            assert torch.equal(kq, ck) and torch.equal(ks, sk[:, 0]) and torch.equal(kb, bk[:, 0])
            assert torch.equal(vq, cv) and torch.equal(vs, sv[..., 0]) and torch.equal(vb, bv[..., 0])


@pytest.mark.parametrize("G", [1, 4, 7])
@pytest.mark.parametrize("bits", [4, 8])
def test_decode_against_sdpa_and_the_oracle(bits, G):
    """Decode after each of 40 appends (crossing page boundaries, a partial page most of the time):
    SDPA over the dequantized cache within rel-norm 1e-5 (tests/test_cpu.py:79-96), and the oracle's
    output within 1e-5 (the product folds the scales into q and the softmax weights: another fp32
    summation order)."""
    torch.manual_seed(G * 10 + bits)
    H, D, B = 2, 128, 3
    prod = cpu_cache(1, H, H * G, D, batch_size=B, bits=bits)
    orc = oracle_cache(1, H, H * G, D, batch_size=B, bits=bits)
    K, V = torch.randn(B, H, 45, D), torch.randn(B, H, 45, D)
    K[..., 3] += 40
    for c in (prod, orc):
        c.write(0, K, V)
    for _ in range(40):
        k, v, q = torch.randn(B, H, 1, D), torch.randn(B, H, 1, D), torch.randn(B, H * G, D)
        prod.write(0, k, v)
        orc.write(0, k, v)
        out, want = prod.attend(0, q), orc.attend(0, q)
        hk, hv = prod.dequantize(0)
        ref = F.scaled_dot_product_attention(q[:, :, None], hk, hv, enable_gqa=G > 1)[:, :, 0]
        assert (out - ref).norm() / ref.norm() < 1e-5
        assert (out - want).norm() / want.norm() < 1e-5
    assert torch.equal(prod.pool, orc.pool)


@pytest.mark.parametrize("n", [0, 31, 32, 200])
def test_attend_chunk_blockwise(n):
    """History in one-page blocks + tail + causal chunk == one masked SDPA over everything
    (tests/test_cpu.py:207-222)."""
    torch.manual_seed(n)
    B, H, G, D, T = 2, 2, 3, 64, 37
    c = cpu_cache(1, H, H * G, D, batch_size=B, bits=4)
    if n:
        c.write(0, torch.randn(B, H, n, D), torch.randn(B, H, n, D))
    q, k, v = torch.randn(B, H * G, T, D), torch.randn(B, H, T, D), torch.randn(B, H, T, D)
    out = c.attend_chunk(0, q, k, v, block_bytes=1)
    hk, hv = c.dequantize(0)
    K, V = torch.cat([hk, k], 2), torch.cat([hv, v], 2)
    mask = torch.ones(T, n + T, dtype=torch.bool).tril(diagonal=n)
    ref = F.scaled_dot_product_attention(q, K.repeat_interleave(G, 1), V.repeat_interleave(G, 1),
                                         attn_mask=mask, scale=c.scale)
    assert (out - ref).norm() / ref.norm() < 1e-5


@pytest.mark.parametrize("D,G", [(64, 3), (128, 4), (256, 2)])
@pytest.mark.parametrize("bits", [4, 8])
def test_ragged_sessions(bits, D, G):
    """The vLLM-style ragged simulation of the oracle tests (tests/test_ragged.py:139-151) on the product's
    CPU Ops: scattered blocks of a padded pool, a padded table, strided V rows, decodes and chunks mixed;
    every step's records checked against the reference test's quantization, tails exact, attention
    against float64."""
    torch.manual_seed(0)
    rng = random.Random(2)
    host = RaggedHost(D, bits, H=2, G=G, n_req=5)
    host.ops = Ops(torch.device("cpu"), D, bits, G, torch.float32)
    host.step([0, 1, 2], [70, 33, 5])
    host.step([3, 4], [31, 64])
    for _ in range(25):
        dec = [r for r in range(5) if rng.random() < 0.7]
        chk = [r for r in range(5) if r not in dec and rng.random() < 0.5]
        if dec or chk:
            host.step(dec + chk, [1] * len(dec) + [rng.randint(2, 40) for _ in chk])


@pytest.mark.parametrize("D", [64, 128, 256])
def test_fwht_equals_the_oracle(D):
    torch.manual_seed(D)
    x = torch.randn(77, D) * torch.logspace(-3, 3, D)
    prod, orc = Ops("cpu", D, 4, 1, torch.float32), OracleOps("cpu", D, 4, 1)
    a, b = prod.fwht(x), orc.fwht(x)
    assert torch.equal(a, b)
    y = x.clone()
    assert prod.fwht(y, out=y) is y and torch.equal(y, a)            # in place
    assert torch.allclose(a, x @ hadamard(D, "cpu"), rtol=1e-5, atol=1e-4 * float(x.abs().max()))


@pytest.mark.parametrize("rot", [False, True])
@pytest.mark.parametrize("D,bits", [(64, 4), (128, 8), (256, 4)])
def test_unpack_equals_the_oracle(D, bits, rot):
    """One packed-prefill group (full pages, partial pages with K from the tails, new rows) through the
    product's and the oracle's unpack: identical keys and values."""
    g = torch.Generator().manual_seed(D + bits + rot)
    H, blocks = 2, 20
    cache = torch.randint(0, 256, (blocks, H, record_bytes(D, bits)), generator=g, dtype=torch.uint8)
    hv = cache.view(blocks, H, -1)[..., 2 * PAGE * (D if bits == 8 else D // 2):].view(torch.float16)
    hv.copy_(torch.rand(hv.shape, generator=g).half() * 0.1)       # finite scales and biases
    tail_k = torch.randn(5, H, PAGE, D, generator=g)
    page_blk = torch.tensor([3, 7, 11, 0], dtype=torch.int32)
    page_dst = torch.tensor([0, 64, 32, 100], dtype=torch.int32)
    tail_blk = torch.tensor([5, 9], dtype=torch.int32)
    tail_info = torch.tensor([[132, 7, 2], [96, 4, 4]], dtype=torch.int32).reshape(-1)
    k_new, v_new = torch.randn(6, H, D, generator=g), torch.randn(6, H, D, generator=g)
    new_dst = torch.tensor([139, 140, 141, 142, 143, 144], dtype=torch.int32)
    outs = []
    for ops in (Ops("cpu", D, bits, 1, torch.float32), OracleOps("cpu", D, bits, 1)):
        kp, vp = torch.full((150, H, D), float("nan")), torch.full((150, H, D), float("nan"))
        ops.unpack(cache, page_blk, page_dst, tail_blk, tail_info, tail_k, k_new, v_new, new_dst, kp, vp, rot)
        outs.append((kp, vp))
    (ka, va), (kb, vb) = outs
    assert torch.equal(ka.nan_to_num(7.0), kb.nan_to_num(7.0)) and torch.equal(va.nan_to_num(7.0), vb.nan_to_num(7.0))
    assert not ka[:145].isnan().any() and not va[:145].isnan().any()          # every named row written
    assert ka[145:].isnan().all() and va[145:].isnan().all()                  # the others untouched


def test_cpu_cache_serves_the_c1_case():
    """The reference's CPU-runnable configuration (batch 1, 8 q / 2 kv heads, D 128, 512 tokens, int4,
    rotation on) through KushCache on the CPU path: prefill in chunks, 16 decode steps, each output
    within 1e-5 of the oracle-backed cache's."""
    torch.manual_seed(11)
    H, G, D, N = 2, 4, 128, 512
    prod = cpu_cache(1, H, H * G, D, batch_size=1, bits=4, rotate=True)
    orc = oracle_cache(1, H, H * G, D, batch_size=1, bits=4, rotate=True)
    K, V = torch.randn(1, H, N, D), torch.randn(1, H, N, D)
    for a in range(0, N, 200):
        q = torch.randn(1, H * G, min(200, N - a), D)
        outs = [c.attend_chunk(0, q, K[:, :, a:a + 200], V[:, :, a:a + 200]) for c in (prod, orc)]
        for c in (prod, orc):
            c.write(0, K[:, :, a:a + 200], V[:, :, a:a + 200])
        assert (outs[0] - outs[1]).norm() / outs[1].norm() < 1e-5
    for _ in range(16):
        k, v, q = torch.randn(1, H, 1, D), torch.randn(1, H, 1, D), torch.randn(1, H * G, D)
        for c in (prod, orc):
            c.write(0, k, v)
        a, b = prod.attend(0, q), orc.attend(0, q)
        assert (a - b).norm() / b.norm() < 1e-5
    assert torch.equal(prod.pool, orc.pool)
