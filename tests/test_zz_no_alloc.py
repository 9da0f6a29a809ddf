"""kush_decode_noalloc (needs an MI355X): the allocation-free decode, called through the C ABI, gives
the same bits as kush_decode_ex with caller-owned split-K buffers on the same inputs -- the same
kernels, split ranges and waves, only the partials and counters live in the library's static device
array -- on calls in a row whose second is smaller (fewer sequences and splits), so the array keeps
the last call's contents and its counters must have reset themselves. Both are also checked against
the CPU oracle (max-abs 2e-3 plus the output's rounding, per element). A request beyond the array's
stated maximum is rejected before any launch. Covered launch shapes: shared splits at 4 and 8 waves;
wave splits (each of 4 waves a split of its own, the workgroup's merge of its 4 splits in LDS, then
the last workgroup's over NS / 4 partials); more than 16 q heads per kv head (a merge counter per head
chunk); a rotated cache. No counterpart in the reference."""
import pytest
import torch

import kushkash_amd as kk
from _harness import assert_out_close
from kushkash_amd import _lib
from kushkash_amd._ops import DTYPE_CODE, PAGE, _byte_strides
from oracle.cpu_ops import OracleOps

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
D, BITS, G, H, DTYPE = 128, 4, 4, 2, torch.bfloat16


def _cache(lens, seed, g=G, h=H, rot=False):
    torch.manual_seed(seed)
    S, G, H = len(lens), g, h
    ops = kk.Ops(torch.device(DEV), D, BITS, G, DTYPE)
    pages = max(1, -(-max(lens) // PAGE))
    cache = torch.zeros(S * pages, H, kk.record_bytes(D, BITS), dtype=torch.uint8, device=DEV)
    bt = torch.randperm(S * pages, dtype=torch.int32).view(S, pages).to(DEV)
    tail_k = torch.zeros(S, H, PAGE, D, dtype=DTYPE, device=DEV)
    tail_idx = torch.arange(S, dtype=torch.int32, device=DEV)
    n = sum(lens)
    k = torch.randn(n, H, D, dtype=DTYPE, device=DEV)
    v = torch.randn(n, H, D, dtype=DTYPE, device=DEV)
    qsl = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(S)], dtype=torch.int32, device=DEV)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    jobs = [(s, p) for s in range(S) for p in range(-(-lens[s] // PAGE))]
    js = torch.tensor([j[0] for j in jobs], dtype=torch.int32, device=DEV)
    jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32, device=DEV)
    ops.write(k, v, qsl, seq_lens, tail_idx, js, jp, cache, bt, tail_k, fused=True, rot=rot)
    return cache, bt, tail_k, tail_idx, seq_lens, G, H, int(rot)


def _decode(noalloc: bool, state, q, ns, waves):
    cache, bt, tail_k, tail_idx, seq_lens, G, H, rot = state
    S = q.shape[0]
    bs, hs = _byte_strides(cache)
    out = torch.full_like(q, float("nan"))
    st = torch.cuda.current_stream().cuda_stream
    head = (D, BITS, G, DTYPE_CODE[DTYPE], q.data_ptr(), out.data_ptr(), cache.data_ptr(), bs, hs, tail_k.data_ptr(),
            tail_idx.data_ptr(), bt.data_ptr(), seq_lens.data_ptr(), bt.stride(0), H, D ** -0.5, ns)
    if noalloc:
        print(f"kush_decode_noalloc S={S} G={G} H={H} ns={ns} waves={waves} rot={rot}", flush=True)
        _lib.call("kush_decode_noalloc", *head, S, st, bt.shape[1], waves, None, rot)
    else:
        rows = S * H * ns * G
        work = torch.empty(rows * (D + 2), dtype=torch.float32, device=DEV)
        sync = torch.zeros(S * H * -(-G // 16), dtype=torch.int32, device=DEV)
        part = (work.data_ptr(), work.data_ptr() + rows * 2 * 4) if ns > 1 else (None, None)
        _lib.call("kush_decode_ex", *head, *part, S, st, bt.shape[1], sync.data_ptr() if ns > 1 else None, waves,
                  None, rot)
    torch.cuda.synchronize()
    return out.cpu()


def _oracle(state, q):
    cache, bt, tail_k, tail_idx, seq_lens, G, _, _ = state
    want = torch.empty(q.shape)
    OracleOps("cpu", D, BITS, G).decode(q.float().cpu(), want, cache.cpu(), bt.cpu(), seq_lens.cpu(), tail_idx.cpu(),
                                        tail_k.float().cpu(), D ** -0.5)
    return want


@pytest.mark.parametrize("waves", [4, 8])
def test_noalloc_matches_caller_buffers_on_calls_in_a_row(waves):
    big = _cache([1, 40 * PAGE, 0, 17 * PAGE + 5, 3 * PAGE, 31, 63 * PAGE + 1], seed=5)
    small = _cache([9 * PAGE + 2, PAGE], seed=6)
    g = torch.Generator().manual_seed(waves)
    q_big = torch.randn(7, H * G, D, generator=g).to(DTYPE).to(DEV)
    q_small = torch.randn(2, H * G, D, generator=g).to(DTYPE).to(DEV)
    # (state, q, splits): large, then smaller (fewer sequences and splits), then one split (no
    # scratch), then the large one again
    for i, (state, q, ns) in enumerate([(big, q_big, 16), (small, q_small, 3), (small, q_small, 1), (big, q_big, 16)]):
        got = _decode(True, state, q, ns, waves)
        ref = _decode(False, state, q, ns, waves)
        assert torch.equal(got, ref), f"call {i}: noalloc differs from kush_decode_ex"
        assert_out_close(got, _oracle(state, q), DTYPE, what=f"call {i} vs oracle")


@pytest.mark.parametrize("g, rot", [(20, False), (4, True)])
def test_noalloc_wave_splits_head_chunks_and_rotation(monkeypatch, g, rot):
    """Wave splits forced on (the in-LDS merge of a workgroup's 4 splits into one partial, then the last
    workgroup's merge over NS / 4 partials, in the static array), with 20 q heads per kv head (two head
    chunks, a merge counter each) or a rotated cache; calls in a row, the second smaller."""
    monkeypatch.setenv("KUSHKASH_AMD_WAVE_SPLITS", "1")
    h = 1 if g > 16 else H
    big = _cache([40 * PAGE + 7, 3 * PAGE, 64 * PAGE, 0, 17 * PAGE + 30], seed=7, g=g, h=h, rot=rot)
    small = _cache([9 * PAGE + 2, 21 * PAGE], seed=8, g=g, h=h, rot=rot)
    gen = torch.Generator().manual_seed(g)
    q_big = torch.randn(5, h * g, D, generator=gen).to(DTYPE).to(DEV)
    q_small = torch.randn(2, h * g, D, generator=gen).to(DTYPE).to(DEV)
    for i, (state, q, ns) in enumerate([(big, q_big, 16), (small, q_small, 8), (big, q_big, 16)]):
        got = _decode(True, state, q, ns, 4)
        ref = _decode(False, state, q, ns, 4)
        assert torch.equal(got, ref), f"call {i}: noalloc differs from kush_decode_ex"
        if not rot:
            assert_out_close(got, _oracle(state, q), DTYPE, what=f"call {i} vs oracle")
        else:                                    # the same launches without wave splits: same values, to rounding
            monkeypatch.setenv("KUSHKASH_AMD_WAVE_SPLITS", "0")
            shared = _decode(False, state, q, ns, 4)
            monkeypatch.setenv("KUSHKASH_AMD_WAVE_SPLITS", "1")
            assert_out_close(got, shared.float(), DTYPE, base=1e-3, what=f"call {i} vs shared splits")


def test_noalloc_rejects_requests_beyond_its_maximum():
    # 4096 sequences x 8 kv heads x 256 splits x 4 heads: ~4.4 GB of partials, far past 64 MiB; rejected
    # before anything is launched (the pointers are never read)
    lib = _lib.lib()
    rc = lib.kush_decode_noalloc(D, BITS, G, DTYPE_CODE[DTYPE], None, None, None, 0, 0, None, None, None, None, 0, 8,
                                 1.0, 256, 4096, None, 0, 4, None, 0)
    assert rc == -2
    msg = lib.kush_last_error().decode()
    assert "maximum" in msg and "kush_decode_ex" in msg, msg
    with pytest.raises(RuntimeError, match="kush_decode_noalloc failed"):
        _lib.call("kush_decode_noalloc", D, BITS, G, DTYPE_CODE[DTYPE], None, None, None, 0, 0, None, None, None,
                  None, 0, 8, 1.0, 256, 4096, None, 0, 4, None, 0)
