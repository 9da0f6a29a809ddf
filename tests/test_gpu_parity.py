"""GPU parity against the CPU oracle (needs an MI355X): packed records and K tails bit-exact, decode
outputs within tolerance. Mirrors the reference's tests/test_gpu.py (test_pages_match_cpu,
test_decode_matches_reference, test_split_k_long_context) with the oracle as the CPU side."""
import pytest
import torch
import torch.nn.functional as F

import kushkash_amd as kk
from _harness import assert_out_close, oracle_cache
from kushkash_amd._ops import PAGE
from oracle.cpu_ops import OracleOps

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _fill(c, K, V, bulk: int) -> None:
    """Bulk write of the first `bulk` tokens, then one append per token (the reference's pattern)."""
    T = K.shape[2]
    if bulk:
        c.write(0, K[:, :, :bulk], V[:, :, :bulk])
    for t in range(bulk, T):
        c.write(0, K[:, :, t:t + 1], V[:, :, t:t + 1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_pages_match_oracle(D, bits, dtype):
    """Record bytes and K tails of bulk writes + token appends are identical to the oracle's
    (reference: tests/test_gpu.py:14-33); K channel 1 carries a +50 offset."""
    torch.manual_seed(D + bits)
    B, H, T = 2, 2, 3 * PAGE + 5
    K, V = torch.randn(B, H, T, D) * 2, torch.randn(B, H, T, D)
    K[..., 1] += 50
    K, V = K.to(dtype), V.to(dtype)
    g = kk.KushCache(1, H, H, D, batch_size=B, bits=bits, device=DEV, dtype=dtype, rotate=False)
    _fill(g, K.to(DEV), V.to(DEV), 40)
    c = oracle_cache(1, H, H, D, batch_size=B, bits=bits, rotate=False)
    _fill(c, K.float(), V.float(), 40)
    n = -(-T // PAGE) * B
    x, y = g.pool[0, :n].cpu(), c.pool[0, :n]
    assert torch.equal(x, y), f"{(x != y).float().mean():.2e} of record bytes differ"
    r = T % PAGE
    assert torch.equal(g.tail_k[0, :, :, :r].float().cpu(), c.tail_k[0, :, :, :r])
    assert torch.equal(g.seq_lens.cpu(), c.seq_lens)


def oracle_decode(c: kk.KushCache, layer: int, q: torch.Tensor) -> torch.Tensor:
    """The oracle's decode over the GPU cache's own records (copied to the CPU), fp32."""
    ops = OracleOps("cpu", c.D, c.bits, c.G)
    out = torch.empty(q.shape, dtype=torch.float32)
    ops.decode(q.float().cpu().contiguous(), out, c.pool[layer].cpu(), c.block_table.cpu(),
               c.seq_lens[layer].cpu(), c.tail_idx.cpu(), c.tail_k[layer].float().cpu(), c.scale)
    return out


CASES = [  # (D, bits, G, dtype, B, N): the reference's CASES (tests/test_gpu.py:36-43)
    (128, 4, 4, torch.float16, 4, 1000), (128, 8, 4, torch.bfloat16, 2, 777),
    (128, 4, 7, torch.bfloat16, 1, 8192), (128, 4, 8, torch.float16, 3, 300),
    (128, 4, 12, torch.float16, 2, 500),
    (64, 4, 4, torch.bfloat16, 2, 2000), (64, 8, 2, torch.float16, 1, 70),
    (256, 4, 2, torch.float16, 2, 1500), (256, 8, 8, torch.bfloat16, 1, 4100),
    (128, 4, 4, torch.float32, 1, 33), (128, 4, 4, torch.float16, 1, 31),
    (128, 8, 20, torch.bfloat16, 2, 200),                                      # G > 16: two head chunks
]


@pytest.mark.parametrize("D,bits,G,dtype,B,N", CASES)
def test_decode_matches_oracle(D, bits, G, dtype, B, N):
    """Decode after every one of the last 8 appends: against the oracle on the same records
    (max-abs 2e-3 + output rounding) and against SDPA over the dequantized cache (rel-norm, the
    reference's tolerances, tests/test_gpu.py:61)."""
    torch.manual_seed(N)
    H = 2
    c = kk.KushCache(2, H, H * G, D, batch_size=B, bits=bits, device=DEV, dtype=dtype, rotate=False)
    K = torch.randn(B, H, N, D, device=DEV, dtype=dtype)
    V = torch.randn(B, H, N, D, device=DEV, dtype=dtype)
    if N > 8:
        c.write(1, K[:, :, :N - 8], V[:, :, :N - 8])
    for t in range(max(0, N - 8), N):
        c.write(1, K[:, :, t:t + 1], V[:, :, t:t + 1])
        q = torch.randn(B, H * G, D, device=DEV, dtype=dtype)
        out = c.attend(1, q).float().cpu()
        want = oracle_decode(c, 1, q)
        assert_out_close(out, want, dtype, what=f"token {t}")
        hk, hv = c.dequantize(1)
        ref = F.scaled_dot_product_attention(q[:, :, None].float(), hk.float(), hv.float(),
                                             enable_gqa=G > 1)[:, :, 0].cpu()
        rel = ((out - ref).norm() / ref.norm()).item()
        assert rel < (2e-2 if dtype == torch.bfloat16 else 3e-3), (t, rel)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("waves", [2, 4, 8])
@pytest.mark.parametrize("ns", [1, 2, 8, 64, 256])
def test_split_k_matches_oracle(ns, waves, fused, monkeypatch):
    """Forced split-K factors incl. splits with no pages (ns > pages), merged inside the decode launch
    (fused: the last workgroup of each sequence / kv head) or by the combine kernel, for every
    waves-per-workgroup variant (reference: tests/test_gpu.py:100-111). Two calls in a row check
    that the merge counters reset themselves."""
    import kushkash_amd._ops as ops_mod
    if not fused:
        monkeypatch.setattr(ops_mod, "SYNC_SLOTS", 0)
    torch.manual_seed(ns)
    B, H, G, D, N = 2, 8, 4, 128, 32 * 100 + 7
    c = kk.KushCache(1, H, H * G, D, batch_size=B, bits=4, device=DEV, dtype=torch.bfloat16, rotate=False)
    K = torch.randn(B, H, N, D, device=DEV, dtype=torch.bfloat16)
    c.write(0, K, K.flip(2))
    work = torch.empty(B * H * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    for call in range(2):
        q = torch.randn(B, H * G, D, device=DEV, dtype=torch.bfloat16)
        out = torch.empty_like(q)
        c.ops.decode(q, out, c.pool[0], c.block_table, c.seq_lens[0], c.tail_idx, c.tail_k[0], c.scale, ns, work,
                     waves=waves)
        want = oracle_decode(c, 0, q)
        assert_out_close(out, want, torch.bfloat16, what=f"call {call}")
    assert int(c.ops._sync.abs().sum()) == 0


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("waves,ns", [(2, 1), (4, 1), (8, 1), (4, 2)])
def test_windows_then_partial_page(bits, waves, ns):
    """A split over more than two 1,024-page windows of block ids that ends in a 13-token partial
    page: the page loop reloads its id table between windows, and the partial page's record goes out
    from inside the last window. Against the oracle."""
    torch.manual_seed(bits * 10 + waves + ns)
    B, H, G, D, N = 1, 2, 4, 128, 32 * 2100 + 13
    c = kk.KushCache(1, H, H * G, D, batch_size=B, bits=bits, device=DEV, dtype=torch.bfloat16, rotate=False)
    K = torch.randn(B, H, N, D, device=DEV, dtype=torch.bfloat16)
    c.write(0, K, K.flip(2))
    work = torch.empty(B * H * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    q = torch.randn(B, H * G, D, device=DEV, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    c.ops.decode(q, out, c.pool[0], c.block_table, c.seq_lens[0], c.tail_idx, c.tail_k[0], c.scale, ns, work,
                 waves=waves)
    assert_out_close(out, oracle_decode(c, 0, q), torch.bfloat16, what=f"{N} tokens")


def test_empty_and_short_sequences():
    """Sequences of 0, 1, 31, 32 and 33 tokens in one batch (ragged lengths through the raw Ops):
    an empty sequence decodes to zeros, as the reference's l = 0 branch."""
    torch.manual_seed(3)
    lens = [0, 1, 31, 32, 33]
    S, H, G, D, bits, dtype = len(lens), 2, 3, 128, 4, torch.bfloat16
    ops = kk.Ops(torch.device(DEV), D, bits, G, dtype)
    pages = 2
    cache = torch.zeros(S * pages, H, kk.record_bytes(D, bits), dtype=torch.uint8, device=DEV)
    bt = torch.randperm(S * pages, dtype=torch.int32).view(S, pages).to(DEV)
    tail_k = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
    tail_idx = torch.arange(S, dtype=torch.int32, device=DEV)
    T = max(lens)
    k = torch.randn(S * T, H, D, dtype=dtype, device=DEV)
    v = torch.randn(S * T, H, D, dtype=dtype, device=DEV)
    qsl = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(S)], dtype=torch.int32, device=DEV)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    jobs = [(s, p) for s in range(S) for p in range(-(-lens[s] // PAGE))]
    js = torch.tensor([j[0] for j in jobs], dtype=torch.int32, device=DEV)
    jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32, device=DEV)
    ops.write(k, v, qsl, seq_lens, tail_idx, js, jp, cache, bt, tail_k)
    q = torch.randn(S, H * G, D, dtype=dtype, device=DEV)
    out = torch.empty_like(q)
    ops.decode(q, out, cache, bt, seq_lens, tail_idx, tail_k, D ** -0.5)
    o = OracleOps("cpu", D, bits, G)
    want = torch.empty(q.shape)
    o.decode(q.float().cpu(), want, cache.cpu(), bt.cpu(), seq_lens.cpu(), tail_idx.cpu(), tail_k.float().cpu(),
             D ** -0.5)
    got = out.float().cpu()
    assert torch.equal(got[0], torch.zeros_like(got[0]))
    assert_out_close(got, want, dtype)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_write_rows_any_stride(bits, dtype, fused):
    """k / v rows whose row stride breaks 16-byte alignment (a free row stride, as the reference's
    _ops.py:6-15 allows) pack the same record bytes and tails as contiguous rows; chunks that start
    mid-page and end mid-page (split K pages, mode-1 tails), then appends with pos_offset -1. The
    second chunks of sequences 0 and 1 complete a page that reads the tail and leave a later page
    partial (the case where the one-launch write's first-page job writes the tail after reading it);
    fused=False runs the reference's two launches."""
    torch.manual_seed(bits)
    S, H, D = 3, 2, 128
    ops = kk.Ops(torch.device(DEV), D, bits, 1, dtype)
    pages = 4
    RB = kk.record_bytes(D, bits)
    bt = torch.randperm(S * pages, dtype=torch.int32).view(S, pages).to(DEV)
    tail_idx = torch.arange(S, dtype=torch.int32, device=DEV)
    lens0, lens1 = [20, 40, 64], [50, 75, 94]                       # two chunks per sequence
    T = max(lens1)
    kf = torch.randn(S * T, H, D) * 3
    vf = torch.randn(S * T, H, D)
    kf[..., 5] += 40

    def packed(stride_pad: int):
        cache = torch.zeros(S * pages, H, RB, dtype=torch.uint8, device=DEV)
        tail_k = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
        big_k = torch.zeros(S * T, H * D + stride_pad, dtype=dtype, device=DEV)
        big_v = torch.zeros(S * T, H * D + stride_pad, dtype=dtype, device=DEV)
        big_k[:, :H * D] = kf.view(S * T, H * D).to(dtype).to(DEV)
        big_v[:, :H * D] = vf.view(S * T, H * D).to(dtype).to(DEV)
        k = big_k[:, :H * D].unflatten(1, (H, D))
        v = big_v[:, :H * D].unflatten(1, (H, D))
        done = [0] * S
        for lens in (lens0, lens1):
            n_new = [lens[s] - done[s] for s in range(S)]
            rows = torch.cat([torch.arange(s * T + done[s], s * T + lens[s]) for s in range(S)]).to(DEV)
            qsl = torch.tensor([0] + [sum(n_new[:i + 1]) for i in range(S)], dtype=torch.int32, device=DEV)
            jobs = [(s, p) for s in range(S) for p in range(done[s] // PAGE, -(-lens[s] // PAGE))]
            js = torch.tensor([j[0] for j in jobs], dtype=torch.int32, device=DEV)
            jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32, device=DEV)
            kr, vr = k[rows], v[rows]                                    # gathered rows, same stride pattern
            if stride_pad:
                kb2 = torch.zeros(kr.shape[0], H * D + stride_pad, dtype=dtype, device=DEV)
                vb2 = torch.zeros(kr.shape[0], H * D + stride_pad, dtype=dtype, device=DEV)
                kb2[:, :H * D] = kr.flatten(1)
                vb2[:, :H * D] = vr.flatten(1)
                kr, vr = kb2[:, :H * D].unflatten(1, (H, D)), vb2[:, :H * D].unflatten(1, (H, D))
            sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
            ops.write(kr, vr, qsl, sl, tail_idx, js, jp, cache, bt, tail_k, fused=fused)
            done = list(lens)
        # appends: one token per sequence at position seq_lens - 1 (vLLM convention)
        for step in range(2):
            sl = torch.tensor([n + 1 + step for n in lens1], dtype=torch.int32, device=DEV)
            ka = torch.randn(S, H, D, generator=torch.Generator().manual_seed(step)).to(dtype)
            va = torch.randn(S, H, D, generator=torch.Generator().manual_seed(10 + step)).to(dtype)
            if stride_pad:
                kb2 = torch.zeros(S, H * D + stride_pad, dtype=dtype, device=DEV)
                vb2 = torch.zeros(S, H * D + stride_pad, dtype=dtype, device=DEV)
                kb2[:, :H * D], vb2[:, :H * D] = ka.flatten(1).to(DEV), va.flatten(1).to(DEV)
                ka, va = kb2[:, :H * D].unflatten(1, (H, D)), vb2[:, :H * D].unflatten(1, (H, D))
            else:
                ka, va = ka.to(DEV), va.to(DEV)
            ops.append(ka, va, sl, tail_idx, cache, bt, tail_k, pos_offset=-1, advance=False)
        torch.cuda.synchronize()
        return cache.cpu(), tail_k.cpu()

    c0, t0 = packed(0)
    c1, t1 = packed(1)                                              # rows 2-byte (bf16) / 4-byte (fp32) off
    assert torch.equal(c0, c1)
    assert torch.equal(t0, t1)
    # and the contiguous rows match the oracle's packing of the same writes
    oc = OracleOps("cpu", D, bits, 1)
    cache = torch.zeros(S * pages, H, RB, dtype=torch.uint8)
    tail_k = torch.zeros(S, H, PAGE, D)
    done = [0] * S
    for lens in (lens0, lens1):
        n_new = [lens[s] - done[s] for s in range(S)]
        rows = torch.cat([torch.arange(s * T + done[s], s * T + lens[s]) for s in range(S)])
        qsl = torch.tensor([0] + [sum(n_new[:i + 1]) for i in range(S)], dtype=torch.int32)
        jobs = [(s, p) for s in range(S) for p in range(done[s] // PAGE, -(-lens[s] // PAGE))]
        oc.write(kf.to(dtype).float()[rows].contiguous(), vf.to(dtype).float()[rows].contiguous(), qsl,
                 torch.tensor(lens, dtype=torch.int32), tail_idx.cpu(),
                 torch.tensor([j[0] for j in jobs], dtype=torch.int32),
                 torch.tensor([j[1] for j in jobs], dtype=torch.int32), cache, bt.cpu(), tail_k)
        done = list(lens)
    for step in range(2):
        sl = torch.tensor([n + 1 + step for n in lens1], dtype=torch.int32)
        ka = torch.randn(S, H, D, generator=torch.Generator().manual_seed(step)).to(dtype).float()
        va = torch.randn(S, H, D, generator=torch.Generator().manual_seed(10 + step)).to(dtype).float()
        oc.append(ka, va, sl, tail_idx.cpu(), cache, bt.cpu(), tail_k, pos_offset=-1, advance=False)
    assert torch.equal(c0, cache)
    assert torch.equal(t0.float(), tail_k)


@pytest.mark.parametrize("ns", [1, 3])
def test_sequence_order_does_not_change_results(ns):
    """Decode with a start order for the sequences (longest first, and a random permutation) gives
    the same bytes as the natural order, with and without split-K."""
    torch.manual_seed(11)
    lens = [5, 300, 64, 1000, 33, 0, 129, 700]
    S, H, G, D, bits, dtype = len(lens), 2, 4, 128, 4, torch.bfloat16
    ops = kk.Ops(torch.device(DEV), D, bits, G, dtype)
    pages = -(-max(lens) // PAGE)
    cache = torch.zeros(S * pages, H, kk.record_bytes(D, bits), dtype=torch.uint8, device=DEV)
    bt = torch.randperm(S * pages, dtype=torch.int32).view(S, pages).to(DEV)
    tail_k = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
    tail_idx = torch.arange(S, dtype=torch.int32, device=DEV)
    n = sum(lens)
    k = torch.randn(n, H, D, dtype=dtype, device=DEV)
    v = torch.randn(n, H, D, dtype=dtype, device=DEV)
    qsl = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(S)], dtype=torch.int32, device=DEV)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    jobs = [(s, p) for s in range(S) for p in range(-(-lens[s] // PAGE))]
    js = torch.tensor([j[0] for j in jobs], dtype=torch.int32, device=DEV)
    jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32, device=DEV)
    ops.write(k, v, qsl, seq_lens, tail_idx, js, jp, cache, bt, tail_k)
    q = torch.randn(S, H * G, D, dtype=dtype, device=DEV)
    work = torch.empty(S * H * ns * G * (D + 2), dtype=torch.float32, device=DEV)

    def run(order):
        out = torch.empty_like(q)
        ops.decode(q, out, cache, bt, seq_lens, tail_idx, tail_k, D ** -0.5, ns, work, order=order)
        torch.cuda.synchronize()
        return out.cpu()

    ref = run(None)                          # 4 waves by the policy: pages go to waves statically
    longest = torch.tensor(sorted(range(S), key=lambda i: -lens[i]), dtype=torch.int32, device=DEV)
    for order in (longest, torch.randperm(S).to(torch.int32).to(DEV)):
        assert torch.equal(run(order), ref)
    # 8 waves sum other page sets per wave than 4 (equal to rounding), but always the same ones
    out8 = [torch.empty_like(q) for _ in range(2)]
    for o8, order in zip(out8, (longest, None)):
        ops.decode(q, o8, cache, bt, seq_lens, tail_idx, tail_k, D ** -0.5, ns, work, waves=8, order=order)
    assert torch.equal(out8[0], out8[1])
    o = OracleOps("cpu", D, bits, G)
    want = torch.empty(q.shape)
    o.decode(q.float().cpu(), want, cache.cpu(), bt.cpu(), seq_lens.cpu(), tail_idx.cpu(), tail_k.float().cpu(),
             D ** -0.5)
    assert_out_close(ref, want, dtype, what="4 waves")
    assert_out_close(out8[0], want, dtype, what="8 waves")


@pytest.mark.parametrize("waves,ns", [(4, 1), (2, 1), (8, 1), (4, 3)])
def test_block_id_prefetch_does_not_change_results(waves, ns):
    """kush_decode through the C ABI with the block table's column count (bt_cols: split 0 fetches its
    first block ids before the length), with 0 (no prefetch) and with a count below the pages in use
    (falls back to reading after the length): the same bytes. The table is a view of a wider one
    (row stride > columns), and the lengths are ragged (0 to 40 pages)."""
    from kushkash_amd import _lib
    from kushkash_amd._ops import DTYPE_CODE, _byte_strides
    torch.manual_seed(17)
    lens = [1, 40 * PAGE, 0, 17 * PAGE + 5, 3 * PAGE, 31]
    S, H, G, D, bits, dtype = len(lens), 2, 4, 128, 4, torch.bfloat16
    ops = kk.Ops(torch.device(DEV), D, bits, G, dtype)
    pages = -(-max(lens) // PAGE)
    cache = torch.zeros(S * pages, H, kk.record_bytes(D, bits), dtype=torch.uint8, device=DEV)
    wide = torch.full((S, pages + 9), -1, dtype=torch.int32, device=DEV)
    wide[:, :pages] = torch.randperm(S * pages, dtype=torch.int32).view(S, pages).to(DEV)
    bt = wide[:, :pages]
    tail_k = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
    tail_idx = torch.arange(S, dtype=torch.int32, device=DEV)
    n = sum(lens)
    k = torch.randn(n, H, D, dtype=dtype, device=DEV)
    v = torch.randn(n, H, D, dtype=dtype, device=DEV)
    qsl = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(S)], dtype=torch.int32, device=DEV)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    jobs = [(s, p) for s in range(S) for p in range(-(-lens[s] // PAGE))]
    js = torch.tensor([j[0] for j in jobs], dtype=torch.int32, device=DEV)
    jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32, device=DEV)
    ops.write(k, v, qsl, seq_lens, tail_idx, js, jp, cache, bt, tail_k)
    q = torch.randn(S, H * G, D, dtype=dtype, device=DEV)
    work = torch.empty(S * H * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    bs, hs = _byte_strides(cache)
    nml = S * H * ns * G * 2

    def run(bt_cols):
        out = torch.empty_like(q)
        _lib.call("kush_decode_ex", D, bits, G, DTYPE_CODE[dtype], q.data_ptr(), out.data_ptr(), cache.data_ptr(), bs,
                  hs, tail_k.data_ptr(), tail_idx.data_ptr(), bt.data_ptr(), seq_lens.data_ptr(), bt.stride(0), H,
                  D ** -0.5, ns, work.data_ptr() if ns > 1 else None, work.data_ptr() + nml * 4 if ns > 1 else None, S,
                  torch.cuda.current_stream().cuda_stream, bt_cols, ops._sync.data_ptr() if ns > 1 else None, waves,
                  None, 0)
        torch.cuda.synchronize()
        return out.cpu()

    ref = run(pages)
    o = OracleOps("cpu", D, bits, G)
    want = torch.empty(q.shape)
    o.decode(q.float().cpu(), want, cache.cpu(), bt.cpu().contiguous(), seq_lens.cpu(), tail_idx.cpu(),
             tail_k.float().cpu(), D ** -0.5)
    assert_out_close(ref, want, dtype)
    for cols in (0, 3):
        assert torch.equal(run(cols), ref), cols           # every wave count sums the same pages in the same order

    # the reference's own argument lists: kush_decode (no prefetch, no in-launch merge, default waves),
    # then kush_combine for split partials -- the reference's two launches (_ops.py:191-213)
    out = torch.empty_like(q)
    st = torch.cuda.current_stream().cuda_stream
    _lib.call("kush_decode", D, bits, G, DTYPE_CODE[dtype], q.data_ptr(), out.data_ptr(), cache.data_ptr(), bs, hs,
              tail_k.data_ptr(), tail_idx.data_ptr(), bt.data_ptr(), seq_lens.data_ptr(), bt.stride(0), H, D ** -0.5,
              ns, work.data_ptr() if ns > 1 else None, work.data_ptr() + nml * 4 if ns > 1 else None, S, st)
    if ns > 1:
        _lib.call("kush_combine", D, G, DTYPE_CODE[dtype], out.data_ptr(), work.data_ptr(), work.data_ptr() + nml * 4,
                  ns, H, S, st)
    torch.cuda.synchronize()
    assert_out_close(out.cpu(), want, dtype)
