"""The write legs of the benchmark configurations at their full sizes (needs an MI355X), byte for
byte against the oracle (the C restatement of the reference's CPU write path, cpu.mojo:248-304, over
the same inputs converted to fp32 -- exact for bf16) from the same starting state:

C4 chunked-prefill write: 8 sequences x 2,048 new tokens, 8 kv heads, D 128, int4, bf16, after a
  131,072-token history -- page-aligned (the C4 configuration) and ending mid-page at a different
  offset per sequence (the first page is completed from the K tail, the last left partial) -- in one
  launch (fused) and as the reference's two (mode 0, then mode 1). Every record the chunk touches
  and every K tail are compared. The history's own records are not materialized: its logical pages
  map to blocks the write never touches, the touched ones to a compact pool whose starting bytes
  (and the tails' rows) are seeded random data, which the write must leave alone or read exactly.
C3 append: 128 sequences of U[256, 8192] tokens (the C3 lengths), 8 kv heads, int8, one new token
  each (pos_offset -1, the serving convention), through the append kernel and through the fused
  append + decode; also with half the sequences completing their page. The real C3 cache is built
  first; the records of the touched pages and the tails are compared with the oracle's append on a
  copy of them, and no other byte of the 1.2 GB cache may change (reference contract:
  tests/test_gpu.py:14-33, pages byte-equal with the CPU path)."""
import math

import pytest
import torch

import bench
import kushkash_amd as kk
from kushkash_amd._ops import PAGE, Ops, pages_touched, record_bytes
from oracle.cpu_ops import OracleOps

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("start", ["page-aligned", "mid-page"])
def test_c4_chunked_write_full_size(start, fused):
    B, Hkv, D, bits, T, HIST = 8, 8, 128, 4, 2048, 131072
    dtype = torch.bfloat16
    offs = [0] * B if start == "page-aligned" else [0, 1, 17, 31, 5, 30, 16, 2]
    n0 = [HIST + o for o in offs]
    total = [n + T for n in n0]
    touched = [pages_touched(a, b) for a, b in zip(n0, total)]
    print(f"C4 write {start} fused={fused}: {sum(len(t) for t in touched)} page jobs x {Hkv} heads", flush=True)
    RB = record_bytes(D, bits)
    g = torch.Generator().manual_seed(4)
    nblk = sum(len(t) for t in touched)
    cache0 = torch.randint(0, 256, (nblk, Hkv, RB), dtype=torch.uint8, generator=g)
    table = torch.zeros(B, max(total) // PAGE + 1, dtype=torch.int32)
    blk = 0
    for i, pages in enumerate(touched):                      # touched pages -> a compact pool, in a seeded order
        ids = torch.randperm(len(pages), generator=g) + blk
        table[i, pages.start:pages.stop] = ids.to(torch.int32)
        blk += len(pages)
    tail0 = torch.randn(B, Hkv, PAGE, D, generator=g).to(dtype)
    k = torch.randn(B * T, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B * T, Hkv, D, generator=g).to(dtype)
    k[:, :, 3] += 6.0                                        # an offset channel, as the C4 keys carry
    qsl = torch.arange(B + 1, dtype=torch.int32) * T
    sl = torch.tensor(total, dtype=torch.int32)
    tail_idx = torch.arange(B, dtype=torch.int32)
    js = torch.tensor([i for i, p in enumerate(touched) for _ in p], dtype=torch.int32)
    jp = torch.tensor([j for p in touched for j in p], dtype=torch.int32)

    ops = Ops(torch.device(DEV), D, bits, 4, dtype)
    cache, tail = cache0.to(DEV), tail0.to(DEV)
    ops.write(k.to(DEV), v.to(DEV), qsl.to(DEV), sl.to(DEV), tail_idx.to(DEV), js.to(DEV), jp.to(DEV), cache,
              table.to(DEV), tail, fused=fused)
    torch.cuda.synchronize()

    want_cache, want_tail = cache0.clone(), tail0.float()
    OracleOps("cpu", D, bits, 4).write(k.float(), v.float(), qsl, sl, tail_idx, js, jp, want_cache, table, want_tail)
    got = cache.cpu()
    if not torch.equal(got, want_cache):
        bad = (got != want_cache).nonzero()
        raise AssertionError(f"{bad.shape[0]} record bytes differ, first at (block, head, byte) {bad[0].tolist()}")
    assert torch.equal(tail.float().cpu(), want_tail), "K tails differ"
    assert not torch.equal(got, cache0)                      # the write did write


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("lens_kind", ["c3", "completing"])
def test_c3_append_full_size(lens_kind, fused):
    B, Hq, Hkv, D, bits = 128, 32, 8, 128, 8
    G, dtype = Hq // Hkv, torch.bfloat16
    lens = torch.randint(256, 8193, (B,), generator=torch.Generator().manual_seed(0)).tolist()
    if lens_kind == "completing":                            # every other new token completes its page
        lens = [n - n % PAGE + PAGE - 1 if i % 2 == 0 else n for i, n in enumerate(lens)]
    print(f"C3 append {lens_kind} fused={fused}: {sum(1 for n in lens if n % PAGE == PAGE - 1)} pages complete",
          flush=True)
    ops = Ops(torch.device(DEV), D, bits, G, dtype)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(0)
    cache, table, tail_k, tail_idx = bench.ragged_cache(ops, lens, 1, Hkv, 6.0, 0.10, gen, DEV)
    k_new = torch.randn(B, Hkv, D, generator=gen, device=DEV).to(dtype)
    v_new = torch.randn(B, Hkv, D, generator=gen, device=DEV).to(dtype)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV) + 1   # the new token is counted (pos = lens[i])

    # the oracle's starting state: the records of each sequence's touched page and all tails
    pg = torch.tensor([n // PAGE for n in lens], dtype=torch.int64, device=DEV)
    blocks = table[torch.arange(B, device=DEV), pg].long()
    small = cache[blocks].cpu()                              # [B, Hkv, RB]
    small_table = torch.zeros(B, max(lens) // PAGE + 1, dtype=torch.int32)
    small_table[torch.arange(B), pg.cpu()] = torch.arange(B, dtype=torch.int32)
    want_tail = tail_k.float().cpu()
    before = cache.clone()

    if fused:
        q = torch.randn(B, Hq, D, generator=gen, device=DEV).to(dtype)
        out = torch.empty_like(q)
        ns = ops.splits(B, Hkv, max(lens) // PAGE + 1)
        work = torch.empty(max(1, B * Hkv * ns * G * (D + 2)), dtype=torch.float32, device=DEV)
        ops.append_decode(k_new, v_new, q, out, cache, table, sl, tail_idx, tail_k, 1.0 / math.sqrt(D), ns, work)
    else:
        ops.append(k_new, v_new, sl, tail_idx, cache, table, tail_k, pos_offset=-1, advance=False)
    torch.cuda.synchronize()

    OracleOps("cpu", D, bits, G).append(k_new.float().cpu(), v_new.float().cpu(), sl.cpu(), tail_idx.cpu(), small,
                                        small_table, want_tail, pos_offset=-1, advance=False)
    got = cache[blocks].cpu()
    if not torch.equal(got, small):
        bad = (got != small).nonzero()
        raise AssertionError(f"{bad.shape[0]} record bytes differ, first at (sequence, head, byte) {bad[0].tolist()}")
    assert torch.equal(tail_k.float().cpu(), want_tail), "K tails differ"
    changed = (cache != before).flatten(1).any(1).nonzero().flatten()
    assert set(changed.tolist()) <= set(blocks.tolist()), "the append wrote outside the touched pages"
    assert torch.equal(sl.cpu(), torch.tensor(lens, dtype=torch.int32) + 1)   # advance = 0: lengths untouched


def test_partial_job_list_takes_the_reference_two_launches():
    """Ops.write with its default (the reference's two launches) accepts any subset of the
    pages_touched jobs, as the reference's write does: with the last touched page's job left out of
    every sequence's list, the records and K tails equal the oracle's write of the same list byte for
    byte (that page's V rows and the new K tail are simply not written); under KUSHKASH_AMD_VALIDATE a
    one-launch write of the same list raises."""
    import os
    B, Hkv, D, bits, T = 4, 2, 128, 4, 70
    dtype = torch.bfloat16
    n0 = [5, 32, 61, 100]
    total = [n + T for n in n0]
    touched = [pages_touched(a, b) for a, b in zip(n0, total)]
    jobs = [(i, p) for i, t in enumerate(touched) for p in list(t)[:-1]]
    RB = record_bytes(D, bits)
    g = torch.Generator().manual_seed(11)
    nblk = max(total) // PAGE + 1
    cache0 = torch.randint(0, 256, (B * nblk, Hkv, RB), dtype=torch.uint8, generator=g)
    table = torch.arange(B * nblk, dtype=torch.int32).view(B, nblk)
    tail0 = torch.randn(B, Hkv, PAGE, D, generator=g).to(dtype)
    k = torch.randn(B * T, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B * T, Hkv, D, generator=g).to(dtype)
    qsl = torch.arange(B + 1, dtype=torch.int32) * T
    sl = torch.tensor(total, dtype=torch.int32)
    tail_idx = torch.arange(B, dtype=torch.int32)
    js = torch.tensor([j[0] for j in jobs], dtype=torch.int32)
    jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32)
    ops = Ops(torch.device(DEV), D, bits, 4, dtype)
    cache, tail = cache0.to(DEV), tail0.to(DEV)
    args = (k.to(DEV), v.to(DEV), qsl.to(DEV), sl.to(DEV), tail_idx.to(DEV), js.to(DEV), jp.to(DEV), cache,
            table.to(DEV), tail)
    ops.write(*args)
    torch.cuda.synchronize()
    want_cache, want_tail = cache0.clone(), tail0.float()
    OracleOps("cpu", D, bits, 4).write(k.float(), v.float(), qsl, sl, tail_idx, js, jp, want_cache, table, want_tail)
    assert torch.equal(cache.cpu(), want_cache), "records differ from the oracle's write of the same jobs"
    assert torch.equal(tail.float().cpu(), want_tail), "K tails differ from the oracle's write of the same jobs"
    if os.environ.get("KUSHKASH_AMD_VALIDATE", "") not in ("", "0"):
        with pytest.raises(ValueError, match="miss touched page"):
            ops.write(*args, fused=True)
