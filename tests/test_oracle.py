"""The CPU oracle (oracle/, the C restatement of the reference CPU path) through the KushCache API
and the raw Ops surface, restating the reference's own CPU tests: codes bit-exact against the
reference test's torch restatement of the format (tests/test_cpu.py:40-76), decode against SDPA
over the dequantized cache (tests/test_cpu.py:79-96), the quantization error bounds
(tests/test_cpu.py:99-106), chunk attention over the history (tests/test_cpu.py:207-222) and the
ragged vLLM-style simulation (tests/test_ragged.py)."""
import random
from dataclasses import dataclass, field

import pytest
import torch
import torch.nn.functional as F

from _harness import oracle_cache, ref_quantize, split_record
from kushkash_amd._ops import (PAGE, as_records, cached_kv, hadamard, history_attention, pages_touched,
                               record_bytes)
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


@dataclass
class _Request:
    """One request of the ragged host: its blocks (logical page order), tail slot, and every token it
    has cached, exactly (the ground truth the stored records and tails are checked against)."""
    slot: int
    blocks: list = field(default_factory=list)
    k: list = field(default_factory=list)            # [H, D] rows, one per cached token
    v: list = field(default_factory=list)

    @property
    def n(self) -> int:
        return len(self.k)


class RaggedHost:
    """A vLLM-like host over the oracle's raw Ops, restating the semantics the reference checks in
    tests/test_ragged.py: blocks taken from a shuffled free list of a pool whose block stride is
    padded, a block table with a padded row stride, tail slots that are a permutation with spares,
    V rows read through a strided view of a fused qkv buffer, and vLLM's positions (seq_lens already
    counts the step's tokens). Each step runs the decodes first (append + decode) and then the
    chunked prefills (attention over history and chunk, then the ragged write)."""

    def __init__(self, D: int, bits: int, H: int, G: int, n_req: int, n_blocks: int = 96, pad: int = 48):
        self.D, self.bits, self.H, self.G = D, bits, H, G
        rb = record_bytes(D, bits)
        storage = torch.zeros(n_blocks, H * rb + pad, dtype=torch.uint8)
        self.pool = storage[:, :H * rb].view(n_blocks, H, PAGE, rb // PAGE)     # strided vLLM-style view
        self.ops = OracleOps("cpu", D, bits, G)
        self.free = random.Random(0).sample(range(n_blocks), n_blocks)
        slots = random.Random(1).sample(range(n_req + 3), n_req)
        self.reqs = [_Request(slot=s) for s in slots]
        self.tail_k = torch.zeros(n_req + 3, H, PAGE, D)
        self.width = 16                                     # block-table columns per request

    # ---------------------------------------------------------------- host bookkeeping
    def _table(self, ids: list) -> torch.Tensor:
        """The requests' block ids as an int32 table view with a padded row stride."""
        t = torch.zeros(len(ids), self.width + 5, dtype=torch.int32)[:, :self.width]
        for row, r in enumerate(ids):
            t[row, :len(self.reqs[r].blocks)] = torch.tensor(self.reqs[r].blocks, dtype=torch.int32)
        return t

    def _grow(self, r: int, total: int) -> None:
        while len(self.reqs[r].blocks) * PAGE < total:
            self.reqs[r].blocks.append(self.free.pop())

    def _stored(self, r: int, n: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The first n tokens of request r as the cache holds them, K, V [H, n, D]."""
        req = self.reqs[r]
        k, v = cached_kv(as_records(self.pool), self._table([r]), n, self.tail_k[req.slot:req.slot + 1], self.D,
                         self.bits, torch.float32)
        return k[0], v[0]

    # ---------------------------------------------------------------- one step
    def step(self, ids: list, qlens: list) -> None:
        H, D, G = self.H, self.D, self.G
        starts = [0]
        for q in qlens:
            starts.append(starts[-1] + q)
        rows = starts[-1]
        k = torch.randn(rows, H, D)
        fused = torch.zeros(rows, 3 * H * D)                 # V lives in the last third of a qkv buffer
        fused[:, 2 * H * D:] = torch.randn(rows, H * D)
        v = fused[:, 2 * H * D:].view(rows, H, D)
        q = torch.randn(rows, H * G, D)
        before = [self.reqs[r].n for r in ids]
        for r, ql in zip(ids, qlens):
            self._grow(r, self.reqs[r].n + ql)
        table = self._table(ids)
        lens = torch.tensor([n + ql for n, ql in zip(before, qlens)], dtype=torch.int32)
        slots = torch.tensor([self.reqs[r].slot for r in ids], dtype=torch.int32)
        n_dec = next((i for i, ql in enumerate(qlens) if ql > 1), len(qlens))     # decodes come first
        out = torch.zeros_like(q)
        expect = {}
        if n_dec:
            self.ops.append(k[:n_dec], v[:n_dec], lens[:n_dec], slots[:n_dec], self.pool, table[:n_dec],
                            self.tail_k, pos_offset=-1, advance=False)
            self.ops.decode(q[:n_dec].contiguous(), out[:n_dec], self.pool, table[:n_dec], lens[:n_dec],
                            slots[:n_dec], self.tail_k, D ** -0.5)
            for i in range(n_dec):                            # the appended token is part of the cache
                expect[i] = self._stored(ids[i], int(lens[i]))
        for i in range(n_dec, len(ids)):
            a, b = starts[i], starts[i + 1]
            hk, hv = self._stored(ids[i], before[i])
            chunk_k, chunk_v = k[a:b].transpose(0, 1), v[a:b].transpose(0, 1)
            expect[i] = (torch.cat([hk, chunk_k], 1), torch.cat([hv, chunk_v], 1))
            slot = self.reqs[ids[i]].slot
            o = history_attention(q[a:b].transpose(0, 1)[None], chunk_k[None], chunk_v[None], as_records(self.pool),
                                  table[i:i + 1], before[i], self.tail_k[slot:slot + 1], D, self.bits, D ** -0.5,
                                  block_bytes=1)
            out[a:b] = o[0].transpose(0, 1)
        if n_dec < len(ids):
            jobs = [(i, pg) for i in range(n_dec, len(ids)) for pg in pages_touched(before[i], int(lens[i]))]
            self.ops.write(k, v, torch.tensor(starts, dtype=torch.int32), lens, slots,
                           torch.tensor([j for j, _ in jobs], dtype=torch.int32),
                           torch.tensor([pg for _, pg in jobs], dtype=torch.int32), self.pool, table, self.tail_k)
        for i, r in enumerate(ids):
            a, b = starts[i], starts[i + 1]
            want = _attention64(q[a:b], *expect[i], G, D ** -0.5)
            err = float((out[a:b].double() - want).norm() / want.norm())
            assert err < 2e-5, (r, before[i], b - a, err)
            self.reqs[r].k += list(k[a:b])
            self.reqs[r].v += list(v[a:b])
            self._check_stored(r)

    def _check_stored(self, r: int) -> None:
        """Tail rows hold the partial page's exact K; every full page's record is the reference test's
        quantization of the exact tokens (codes, scales, biases bit for bit: K per channel over the
        page, V per token), and the partial page's V rows too."""
        req, D, bits = self.reqs[r], self.D, self.bits
        K, V = torch.stack(req.k, 1), torch.stack(req.v, 1)          # [H, n, D]
        full, part = req.n // PAGE, req.n % PAGE
        assert torch.equal(self.tail_k[req.slot, :, :part], K[:, full * PAGE:])
        recs = as_records(self.pool)
        for pg in range(full + (1 if part else 0)):
            kq, ks, kb, vq, vs, vb = split_record(recs[req.blocks[pg]], D, bits)
            n = PAGE if pg < full else part
            rows = slice(pg * PAGE, pg * PAGE + n)
            cv, sv, bv = ref_quantize(V[:, rows], bits, dim=2)
            assert torch.equal(vq[:, :n], cv) and torch.equal(vs[:, :n], sv[..., 0]) and torch.equal(vb[:, :n], bv[..., 0])
            if pg < full:
                ck, sk, bk = ref_quantize(K[:, rows], bits, dim=1)
                assert torch.equal(kq, ck) and torch.equal(ks, sk[:, 0]) and torch.equal(kb, bk[:, 0])


def _attention64(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, G: int, scale: float) -> torch.Tensor:
    """float64 attention of the T queries q [T, H*G, D] -- the last T of the n keys K, V [H, n, D], each
    seeing the keys up to its own position -- as [T, H*G, D]."""
    T, n = q.shape[0], K.shape[1]
    Kx, Vx = K.double().repeat_interleave(G, 0), V.double().repeat_interleave(G, 0)
    s = torch.einsum("thd,hjd->htj", q.double(), Kx) * scale
    visible = torch.arange(n)[None, :] <= (torch.arange(T)[:, None] + n - T)
    s = s.masked_fill(~visible, float("-inf"))
    return torch.einsum("htj,hjd->thd", torch.softmax(s, -1), Vx)


@pytest.mark.parametrize("D,G", [(64, 3), (128, 4)])
@pytest.mark.parametrize("bits", [4, 8])
def test_ragged_mixed_batches(bits, D, G):
    """Chunked prefill and decode mixed in one step over scattered blocks (tests/test_ragged.py:139-151):
    two first steps of chunks of different sizes, then 40 random steps of decodes plus chunks."""
    torch.manual_seed(0)
    rng = random.Random(2)
    host = RaggedHost(D, bits, H=2, G=G, n_req=5)
    host.step([0, 1, 2], [70, 33, 5])
    host.step([3, 4], [31, 64])
    for _ in range(40):
        dec = [r for r in range(5) if rng.random() < 0.7]
        chk = [r for r in range(5) if r not in dec and rng.random() < 0.5]
        if dec or chk:
            host.step(dec + chk, [1] * len(dec) + [rng.randint(2, 40) for _ in chk])


def test_rotation_lowers_attention_error():
    """The point of the rotation: with outlier channels in K and V, decode and chunk attention over
    the int4 cache (oracle backend) land closer to exact attention when the cache rotates
    (tests/test_cpu.py:369-393)."""
    from _rotation_case import rotation_errors
    err = rotation_errors(lambda rot: oracle_cache(1, 2, 8, 128, batch_size=1, bits=4, rotate=rot), "cpu")
    assert err[True][0] < 0.9 * err[False][0] and err[True][1] < 0.9 * err[False][1], err
