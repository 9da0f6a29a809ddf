"""Wave splits (decode_kernel with every one of 4 waves owning a whole split): against the oracle,
against the same launch with the mode switched off (KUSHKASH_AMD_WAVE_SPLITS=0: the waves share each
split's pages; equal to rounding, not in bits, since one wave sums a split's pages in another order
than four waves and their merge), and bitwise against itself on repeated calls. The reference has
no such mode; its split-K tests (tests/test_gpu.py:100-111) are the model."""
import pytest
import torch

import kushkash_amd as kk
from _harness import assert_out_close
from kushkash_amd._ops import PAGE
from oracle.cpu_ops import OracleOps
from test_gpu_append_decode import test_fused_equals_append_then_decode as fused_append_case
from test_gpu_parity import oracle_decode

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _decode(c, q, ns, work, mode, monkeypatch):
    monkeypatch.setenv("KUSHKASH_AMD_WAVE_SPLITS", mode)
    out = torch.empty_like(q)
    print(f"decode ns={ns} waves=4 wave_splits={mode} S={q.shape[0]}", flush=True)
    c.ops.decode(q, out, c.pool[0], c.block_table, c.seq_lens[0], c.tail_idx, c.tail_k[0], c.scale, ns, work,
                 waves=4)
    return out


@pytest.mark.parametrize("bits,dtype,D,G", [(4, torch.bfloat16, 128, 7), (8, torch.float16, 64, 4),
                                            (4, torch.float16, 256, 2), (4, torch.bfloat16, 128, 20)])
@pytest.mark.parametrize("ns,kw", [(8, ""), (16, ""), (64, ""), (8, "2"), (16, "4"), (64, "2"), (64, "8")])
def test_ragged_batch(ns, kw, bits, dtype, D, G, monkeypatch):
    """Ragged lengths (empty, under one page, partial last pages, pages fewer than splits), G > 16
    (two head chunks) included, in the natural and the longest-first start order; two calls in a row
    check that the split counters reset themselves. kw: splits per wave forced (a wave streams its kw
    splits as one run of pages and folds each finished split into its running state; sequences whose
    split length is odd keep one state over the run), else the library's choice."""
    if kw:
        monkeypatch.setenv("KUSHKASH_AMD_SPLITS_PER_WAVE", kw)
    else:
        monkeypatch.delenv("KUSHKASH_AMD_SPLITS_PER_WAVE", raising=False)
    torch.manual_seed(ns * 100 + bits + D + G + len(kw))
    lens = [0, 5, PAGE, 3 * PAGE + 7, 40 * PAGE + 31, 97 * PAGE, 130 * PAGE + 1, 64 * PAGE + 16]
    S, H = len(lens), 2
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
    work = torch.empty(S * H * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    longest = torch.tensor(sorted(range(S), key=lambda i: -lens[i]), dtype=torch.int32, device=DEV)
    o = OracleOps("cpu", D, bits, G)

    def run(q, mode, order=None):
        monkeypatch.setenv("KUSHKASH_AMD_WAVE_SPLITS", mode)
        print(f"decode ns={ns} D={D} bits={bits} G={G} wave_splits={mode} order={order is not None}", flush=True)
        out = torch.empty_like(q)
        ops.decode(q, out, cache, bt, seq_lens, tail_idx, tail_k, D ** -0.5, ns, work, waves=4, order=order)
        torch.cuda.synchronize()
        return out.cpu()

    for call in range(2):
        q = torch.randn(S, H * G, D, dtype=dtype, device=DEV)
        want = torch.empty(q.shape)
        o.decode(q.float().cpu(), want, cache.cpu(), bt.cpu(), seq_lens.cpu(), tail_idx.cpu(), tail_k.float().cpu(),
                 D ** -0.5)
        ws = run(q, "1")
        assert_out_close(ws, want, dtype, what=f"wave splits, call {call}")
        assert_out_close(run(q, "0"), want, dtype, what=f"shared splits, call {call}")
        assert torch.equal(run(q, "1", longest), ws), "wave splits: other bits in another start order"
    assert int(ops._sync.abs().sum()) == 0


@pytest.mark.parametrize("bits,ns,kw", [(4, 8, "1"), (8, 8, "1"), (4, 16, "2"), (8, 32, "4")])
def test_two_windows_per_wave_then_partial_page(bits, ns, kw, monkeypatch):
    """A wave's pages over more than one 256-page window of its own (NS 8 over 2,100 pages: 263 pages
    per split; NS 16 or 32 with 2 or 4 splits per wave: 264 pages per wave, split boundaries inside a
    window and across the window edge) ending in a 13-token partial page, taken by the last wave of
    the last workgroup."""
    monkeypatch.setenv("KUSHKASH_AMD_SPLITS_PER_WAVE", kw)
    torch.manual_seed(bits + ns)
    B, H, G, D, N = 1, 2, 4, 128, 32 * 2100 + 13
    c = kk.KushCache(1, H, H * G, D, batch_size=B, bits=bits, device=DEV, dtype=torch.bfloat16, rotate=False)
    K = torch.randn(B, H, N, D, device=DEV, dtype=torch.bfloat16)
    c.write(0, K, K.flip(2))
    work = torch.empty(B * H * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    q = torch.randn(B, H * G, D, device=DEV, dtype=torch.bfloat16)
    out = _decode(c, q, ns, work, "1", monkeypatch)
    assert_out_close(out, oracle_decode(c, 0, q), torch.bfloat16, what=f"{N} tokens")


@pytest.mark.parametrize("rot", [False, True])
@pytest.mark.parametrize("ns,kw", [(8, "1"), (16, "1"), (16, "2"), (16, "4")])
@pytest.mark.parametrize("D,bits,G,dtype", [(128, 4, 7, torch.bfloat16), (128, 8, 4, torch.float16),
                                            (256, 4, 2, torch.float32)])
def test_fused_append_then_decode(D, bits, G, dtype, ns, kw, rot, monkeypatch):
    """The fused append + decode with wave splits (the workgroup holding the split of the page a
    token completes writes it; with kw splits per wave, the workgroup holding that split among its
    4 kw), rotation folded in or not: the same records, K tails and outputs as the append followed
    by the decode."""
    monkeypatch.setenv("KUSHKASH_AMD_WAVE_SPLITS", "1")
    monkeypatch.setenv("KUSHKASH_AMD_SPLITS_PER_WAVE", kw)
    fused_append_case(D, bits, G, dtype, ns, 4, True, rot, monkeypatch)


def test_policy_takes_four_waves_for_split_counts_that_four_divides():
    """Ops.waves picks 4 waves for NS >= 8 that 4 divides (the library gives every wave a split of its
    own where S * Hkv * ceil(G / 16) * NS / 4 >= 256, kush_decode.hip wave_splits, else the waves
    share each split), and its other rules below that."""
    ops = kk.Ops(torch.device(DEV), 128, 4, 7, torch.bfloat16)
    assert ops.sms == 256
    assert ops.waves(64, 4, 8) == 4 and ops.waves(8, 8, 16) == 4         # wave splits
    assert ops.waves(8, 8, 8) == 4                                       # 128 workgroups: shared splits
    assert ops.waves(64, 8, 10) == 2                                     # 4 does not divide 10
    assert ops.waves(64, 4, 1) == 4 and ops.waves(128, 8, 1) == 2        # C2, C3
