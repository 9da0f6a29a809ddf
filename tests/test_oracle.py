"""The CPU oracle (oracle/, the C restatement of the reference CPU path) through the KushCache API
and the raw Ops surface, restating the reference's own CPU tests: codes bit-exact against the
reference test's torch restatement of the format (tests/test_cpu.py:40-76), decode against SDPA
over the dequantized cache (tests/test_cpu.py:79-96), the quantization error bounds
(tests/test_cpu.py:99-106), chunk attention over the history (tests/test_cpu.py:207-222) and the
ragged vLLM-style simulation (tests/test_ragged.py)."""
import random

import pytest
import torch
import torch.nn.functional as F

from _harness import oracle_cache, ref_dequant, ref_quantize, split_record
from kushkash_amd._ops import (PAGE, as_records, cached_kv, dequant_records, hadamard, history_attention,
                               pages_touched, record_bytes)
from oracle.cpu_ops import OracleOps


@pytest.mark.parametrize("rot", [False, True])
@pytest.mark.parametrize("appends", [False, True])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("bits", [4, 8])
def test_codes_bit_exact(bits, D, appends, rot):
    """Bulk writes and token appends give exactly the reference test's codes and scales (of the
    rotated K and V when the cache rotates: there the rotation's fp32 sums may flip a rounding)."""
    torch.manual_seed(D + bits)
    B, H, T = 2, 3, 3 * PAGE
    c = oracle_cache(1, H, H, D, batch_size=B, bits=bits, rotate=rot)
    K, V = torch.randn(B, H, T, D) * 3, torch.randn(B, H, T, D)
    if appends:
        c.write(0, K[:, :, :40], V[:, :, :40])
        for t in range(40, T):
            c.write(0, K[:, :, t:t + 1], V[:, :, t:t + 1])
    else:
        c.write(0, K, V)
    if rot:
        h = hadamard(D, "cpu")
        K, V = K @ h, V @ h
    for b in range(B):
        for p in range(T // PAGE):
            rec = c.pool[0, int(c.block_table[b, p])]
            kq, ks, kb, vq, vs, vb = split_record(rec, D, bits)
            ck, sk, bk = ref_quantize(K[b, :, p * PAGE:(p + 1) * PAGE], bits, dim=1)
            cv, sv, bv = ref_quantize(V[b, :, p * PAGE:(p + 1) * PAGE], bits, dim=2)
            if rot:
                for got, ref in ((kq, ck), (vq, cv)):
                    d = (got.int() - ref.int()).abs()
                    assert d.max() <= 1 and (d > 0).float().mean() < 1e-3
                for gs, rs, gb, rb in ((ks, sk[:, 0], kb, bk[:, 0]), (vs, sv[..., 0], vb, bv[..., 0])):
                    assert torch.allclose(gs, rs, rtol=2e-3, atol=1e-6)
                    tol = 2e-3 * rb.abs() + 2 ** (bits - 1) * 2e-3 * rs + 1e-6
                    assert bool(((gb - rb).abs() <= tol).all())
                continue
            assert torch.equal(kq, ck) and torch.equal(ks, sk[:, 0]) and torch.equal(kb, bk[:, 0])
            assert torch.equal(vq, cv) and torch.equal(vs, sv[..., 0]) and torch.equal(vb, bv[..., 0])


@pytest.mark.parametrize("G", [1, 4, 7])
@pytest.mark.parametrize("bits", [4, 8])
def test_decode_matches_dequant_reference(bits, G):
    """Decode after each of 70 appends (crossing two page boundaries) equals SDPA over the
    dequantized cache, rel-norm 1e-5; an outlier channel rides along."""
    torch.manual_seed(G * 10 + bits)
    L, H, D, B = 2, 2, 128, 2
    c = oracle_cache(L, H, H * G, D, batch_size=B, bits=bits)
    K, V = torch.randn(B, H, 45, D), torch.randn(B, H, 45, D)
    K[..., 3] += 40
    for layer in range(L):
        c.write(layer, K, V)
    for _ in range(70):
        k, v = torch.randn(B, H, 1, D), torch.randn(B, H, 1, D)
        for layer in range(L):
            c.write(layer, k, v)
        q = torch.randn(B, H * G, D)
        out = c.attend(1, q)
        hk, hv = c.dequantize(1)
        ref = F.scaled_dot_product_attention(q[:, :, None], hk, hv, enable_gqa=G > 1)[:, :, 0]
        assert (out - ref).norm() / ref.norm() < 1e-5


def test_quantization_error_bounds():
    torch.manual_seed(0)
    B, H, D = 1, 2, 128
    for bits, tol in ((8, 0.01), (4, 0.15)):
        c = oracle_cache(1, H, H, D, bits=bits)
        K, V = torch.randn(B, H, 256, D), torch.randn(B, H, 256, D)
        c.write(0, K, V)
        hk, hv = c.dequantize(0)
        assert (hk - K).norm() / K.norm() < tol and (hv - V).norm() / V.norm() < tol


def test_dequantized_error_at_most_half_a_step():
    """Every dequantized value lies within half a quantization step of its input (s / 2 plus the fp32
    rounding of the dequantization), except where the clamp at the top level applies (< 1 step)."""
    torch.manual_seed(1)
    for bits in (4, 8):
        c = oracle_cache(1, 2, 2, 64, bits=bits, rotate=False)
        K, V = torch.randn(1, 2, 64, 64) * 5, torch.randn(1, 2, 64, 64)
        c.write(0, K, V)
        for p in range(2):
            kq, ks, kb, vq, vs, vb = split_record(c.pool[0, int(c.block_table[0, p])], 64, bits)
            kd, vd = kq * ks[:, None] + kb[:, None], vq * vs[..., None] + vb[..., None]
            for x, y, s in ((K[0, :, p * PAGE:(p + 1) * PAGE], kd, ks[:, None]),
                            (V[0, :, p * PAGE:(p + 1) * PAGE], vd, vs[..., None])):
                err = (x - y).abs()
                assert bool((err <= s * 1.0 + 1e-4 * x.abs() + 1e-6).all())
                assert float((err <= s * 0.5 + 1e-4 * x.abs() + 1e-6).float().mean()) > 0.97


@pytest.mark.parametrize("n", [0, 31, 32, 200])
def test_attend_chunk_blockwise(n):
    """History in one-page blocks + tail + causal chunk == one masked SDPA over everything."""
    torch.manual_seed(n)
    B, H, G, D, T = 2, 2, 3, 64, 37
    c = oracle_cache(1, H, H * G, D, batch_size=B, bits=4)
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


def test_decode_threads_agree():
    """The oracle's decode is one independent task per (sequence, kv head): any thread count gives
    bit-identical outputs (the reference's thread pool, cpu.mojo:454-466)."""
    from oracle import cpu_ops
    torch.manual_seed(5)
    c = oracle_cache(1, 4, 16, 128, batch_size=64, bits=4)
    c.write(0, torch.randn(64, 4, 300, 128), torch.randn(64, 4, 300, 128))
    q = torch.randn(64, 16, 128)
    try:
        cpu_ops.set_threads(1)
        one = c.attend(0, q)
        cpu_ops.set_threads(0)
        many = c.attend(0, q)
    finally:
        cpu_ops.set_threads(0)
    assert torch.equal(one, many)


class Sim:
    """Minimal vLLM-like host over the oracle's raw Ops (tests/test_ragged.py:27-135): a block pool
    with a padded block stride, per-request block tables with a padded row stride, permuted tail
    slots, V rows as a strided view into a fused qkv buffer, vLLM positions (seq_lens already counts
    the new tokens)."""

    def __init__(self, D, bits, H, G, n_req, n_blocks=96, max_blocks=16, pad=48):
        self.D, self.bits, self.H, self.G = D, bits, H, G
        rb = record_bytes(D, bits)
        raw = torch.zeros(n_blocks, H * rb + pad, dtype=torch.uint8)
        self.cache = raw[:, :H * rb].view(n_blocks, H, PAGE, rb // PAGE)
        self.ops = OracleOps("cpu", D, bits, G)
        free = list(range(n_blocks))
        random.Random(0).shuffle(free)
        self.free = free
        self.bt = torch.zeros(n_req, max_blocks, dtype=torch.int32)
        self.lens = [0] * n_req
        self.tail_idx = torch.tensor(random.Random(1).sample(range(n_req + 3), n_req), dtype=torch.int32)
        self.tail_k = torch.zeros(n_req + 3, H, PAGE, D)
        self.exact = [(torch.zeros(H, 0, D), torch.zeros(H, 0, D)) for _ in range(n_req)]

    def ensure_blocks(self, r, total):
        for p in range(-(-total // PAGE)):
            if p >= -(-self.lens[r] // PAGE):
                self.bt[r, p] = self.free.pop()

    def history(self, r, n):
        ts = int(self.tail_idx[r])
        k, v = cached_kv(as_records(self.cache), self.bt[r:r + 1], n, self.tail_k[ts:ts + 1], self.D, self.bits,
                         torch.float32)
        return k[0], v[0]

    def step(self, reqs, qlens):
        rows_k, rows_v, qsl, seq_lens = [], [], [0], []
        for r, ql in zip(reqs, qlens):
            rows_k.append(torch.randn(ql, self.H, self.D))
            rows_v.append(torch.randn(ql, self.H, self.D))
            qsl.append(qsl[-1] + ql)
            self.ensure_blocks(r, self.lens[r] + ql)
            seq_lens.append(self.lens[r] + ql)
        k_all = torch.cat(rows_k)
        qkv = torch.zeros(k_all.shape[0], 3 * self.H * self.D)
        qkv[:, 2 * self.H * self.D:] = torch.cat(rows_v).flatten(1)
        v_all = qkv[:, 2 * self.H * self.D:].view(-1, self.H, self.D)
        q_all = torch.randn(k_all.shape[0], self.H * self.G, self.D)
        W = self.bt.shape[1]
        bt = torch.zeros(len(reqs), W + 7, dtype=torch.int32)[:, :W]
        bt[:] = self.bt[reqs]
        sl = torch.tensor(seq_lens, dtype=torch.int32)
        ti = self.tail_idx[reqs].contiguous()
        nd = next((i for i, ql in enumerate(qlens) if ql != 1), len(qlens))
        outs = torch.empty_like(q_all)
        refs = {}
        if nd:
            self.ops.append(k_all[:nd], v_all[:nd], sl[:nd], ti[:nd], self.cache, bt[:nd], self.tail_k,
                            pos_offset=-1, advance=False)
            self.ops.decode(q_all[:nd].contiguous(), outs[:nd], self.cache, bt[:nd], sl[:nd], ti[:nd],
                            self.tail_k, self.D ** -0.5)
            for i in range(nd):
                refs[i] = self.history(reqs[i], seq_lens[i])
        rec = as_records(self.cache)
        for i in range(nd, len(reqs)):
            r, a, b = reqs[i], qsl[i], qsl[i + 1]
            ts = int(ti[i])
            hk, hv = self.history(r, self.lens[r])
            refs[i] = (torch.cat([hk, k_all[a:b].permute(1, 0, 2)], 1),
                       torch.cat([hv, v_all[a:b].permute(1, 0, 2)], 1))
            o = history_attention(q_all[a:b].permute(1, 0, 2).unsqueeze(0), k_all[a:b].permute(1, 0, 2).unsqueeze(0),
                                  v_all[a:b].permute(1, 0, 2).unsqueeze(0), rec, bt[i:i + 1], self.lens[r],
                                  self.tail_k[ts:ts + 1], self.D, self.bits, self.D ** -0.5, block_bytes=1)
            outs[a:b] = o[0].permute(1, 0, 2)
        if nd < len(reqs):
            jobs = [(i, p) for i in range(nd, len(reqs)) for p in pages_touched(self.lens[reqs[i]], seq_lens[i])]
            js = torch.tensor([j[0] for j in jobs], dtype=torch.int32)
            jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32)
            self.ops.write(k_all, v_all, torch.tensor(qsl, dtype=torch.int32), sl, ti, js, jp, self.cache, bt,
                           self.tail_k)
        for i, r in enumerate(reqs):
            a, b = qsl[i], qsl[i + 1]
            K, V = refs[i]
            mask = torch.ones(b - a, K.shape[1], dtype=torch.bool).tril(diagonal=K.shape[1] - (b - a))
            ref = F.scaled_dot_product_attention(q_all[a:b].permute(1, 0, 2), K.repeat_interleave(self.G, 0),
                                                 V.repeat_interleave(self.G, 0), attn_mask=mask)
            err = (outs[a:b] - ref.permute(1, 0, 2)).norm() / ref.norm()
            assert err < 2e-5, (r, self.lens[r], b - a, float(err))
            self.lens[r] = seq_lens[i]
        for i, r in enumerate(reqs):                 # stored state == ground truth
            a, b = qsl[i], qsl[i + 1]
            ek, ev = self.exact[r]
            ek = torch.cat([ek, k_all[a:b].permute(1, 0, 2)], 1)
            ev = torch.cat([ev, v_all[a:b].permute(1, 0, 2)], 1)
            self.exact[r] = (ek, ev)
            n = seq_lens[i]
            ts, rr, full = int(self.tail_idx[r]), n % PAGE, n // PAGE
            assert torch.equal(self.tail_k[ts, :, :rr], ek[:, full * PAGE:])
            if rr:
                v = dequant_records(as_records(self.cache)[self.bt[r, full].long()], self.D, self.bits,
                                    torch.float32)[1]
                assert torch.allclose(v[:, :rr], ref_dequant(ev[:, full * PAGE:], self.bits, 2), atol=1e-5)
            if full:
                k, v = dequant_records(as_records(self.cache)[self.bt[r, :full].long()], self.D, self.bits,
                                       torch.float32)
                rk = ref_dequant(ek[:, :full * PAGE].reshape(self.H, full, PAGE, self.D).transpose(0, 1), self.bits, 2)
                rv = ref_dequant(ev[:, :full * PAGE].reshape(self.H, full, PAGE, self.D).transpose(0, 1), self.bits, 3)
                assert torch.allclose(k, rk, atol=1e-5) and torch.allclose(v, rv, atol=1e-5)


@pytest.mark.parametrize("D,G", [(64, 3), (128, 4)])
@pytest.mark.parametrize("bits", [4, 8])
def test_ragged_mixed_batches(bits, D, G):
    """Chunked prefill and decode mixed in one step over scattered blocks (tests/test_ragged.py:139-151)."""
    torch.manual_seed(0)
    rng = random.Random(2)
    sim = Sim(D, bits, H=2, G=G, n_req=5)
    sim.step([0, 1, 2], [70, 33, 5])
    sim.step([3, 4], [31, 64])
    for _ in range(40):
        dec = [r for r in range(5) if rng.random() < 0.7]
        chk = [r for r in range(5) if r not in dec and rng.random() < 0.5]
        if not dec + chk:
            continue
        sim.step(dec + chk, [1] * len(dec) + [rng.randint(2, 40) for _ in chk])


def test_rotation_lowers_attention_error():
    """The point of the rotation: with outlier channels in K and V, decode and chunk attention over
    the int4 cache (oracle backend) land closer to exact attention when the cache rotates
    (tests/test_cpu.py:369-393)."""
    from _rotation_case import rotation_errors
    err = rotation_errors(lambda rot: oracle_cache(1, 2, 8, 128, batch_size=1, bits=4, rotate=rot), "cpu")
    assert err[True][0] < 0.9 * err[False][0] and err[True][1] < 0.9 * err[False][1], err
