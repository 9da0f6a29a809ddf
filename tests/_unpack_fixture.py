"""Inputs for the packed-prefill unpack tests (CPU and GPU), and a torch restatement of the
reference test's fp64 unpack oracle (kushkash/_ops.py:398-436, used by tests/test_cpu.py:458-477
and tests/test_gpu.py:221-240).

make_group builds one packed group the way the reference's fixture (tests/_unpack_case.py) shapes
it: random record bytes with sane fp16 scales and biases, full history pages, partial pages with
1..31 tokens (K in distinct tail slots), and new rows in runs, with never-written gap rows between
groups so a test can see that nothing else is touched."""
from __future__ import annotations

import torch

from _harness import split_record
from kushkash_amd._ops import PAGE, fwht_reference, record_bytes

INDEX_NAMES = ("page_blk", "page_dst", "tail_blk", "tail_info", "tail_k", "k_new", "v_new", "new_dst")


def make_group(D: int, bits: int, dtype: torch.dtype, *, seed: int = 0, H: int = 2, n_pages: int = 5,
               tail_tokens=(1, 17, 31), new_runs=(20, 25), slots: int = 4, spare_blocks: int = 4) -> dict:
    g = torch.Generator().manual_seed(seed)
    n_tail = len(tail_tokens)
    n_blk = n_pages + n_tail + spare_blocks
    dc = D if bits == 8 else D // 2
    rec = torch.randint(0, 256, (n_blk, H, record_bytes(D, bits)), dtype=torch.uint8, generator=g)
    meta = rec[:, :, 2 * PAGE * dc:].view(torch.float16)            # [n_blk, H, 2D + 2P]
    meta[..., :D] = (torch.rand(n_blk, H, D, generator=g) * 0.1).half()                     # K scales
    meta[..., D:2 * D] = ((torch.rand(n_blk, H, D, generator=g) - 0.5) * 0.4).half()        # K biases
    meta[..., 2 * D:2 * D + PAGE] = (torch.rand(n_blk, H, PAGE, generator=g) * 0.1).half()  # V scales
    meta[..., 2 * D + PAGE:] = ((torch.rand(n_blk, H, PAGE, generator=g) - 0.5) * 0.4).half()
    blocks = torch.randperm(n_blk, generator=g)
    row, gaps = 0, []

    def gap():
        nonlocal row
        gaps.append(row)
        row += 1

    page_dst = []
    for i in range(n_pages):                                         # a gap row after every third page
        page_dst.append(row)
        row += PAGE
        if i % 3 == 2:
            gap()
    tail_slot = torch.randperm(slots, generator=g)[:n_tail].tolist()
    info = []
    for i, n in enumerate(tail_tokens):
        info += [row, n, tail_slot[i]]
        row += n
        if i == 0:
            gap()
    new_dst = []
    for n in new_runs:
        new_dst += list(range(row, row + n))
        row += n
        gap()
    n_new = len(new_dst)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32)
    return dict(records=rec, page_blk=blocks[:n_pages].to(torch.int32), page_dst=i32(page_dst),
                tail_blk=blocks[n_pages:n_pages + n_tail].to(torch.int32), tail_info=i32(info),
                tail_k=(torch.randn(slots, H, PAGE, D, generator=g) * 0.5).to(dtype),
                k_new=torch.randn(n_new, H, D, generator=g).to(dtype), v_new=torch.randn(n_new, H, D, generator=g).to(dtype),
                new_dst=i32(new_dst), rows=row + 1, H=H, gaps=gaps + [row])


def unpack_torch(c: dict, D: int, bits: int, rot: bool, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """kp, vp of group c (NaN where nothing is written): dequantization in fp64 rounded once to fp32
    (equal to the kernels' fp32 fma(code, scale, bias): code * scale is exact, and the fp64 sum of
    fp16-scaled terms of similar magnitude is too), then the canonical rotation, then one rounding
    to dtype. Follows the reference test's oracle, kushkash/_ops.py:398-436."""
    H, rows = c["H"], c["rows"]
    kp = torch.full((rows, H, D), float("nan"), dtype=dtype)
    vp = kp.clone()
    kq, ks, kb, vq, vs, vb = split_record(c["records"], D, bits)     # codes [blk, H, 32, D]

    def dequant(blk):
        k = (kq[blk].double() * ks[blk, :, None, :].double() + kb[blk, :, None, :].double()).float()
        v = (vq[blk].double() * vs[blk, :, :, None].double() + vb[blk, :, :, None].double()).float()
        return k, v                                                   # [H, 32, D] fp32

    def put(r, k, v):                                                 # k, v [H, D] fp32
        if rot:
            k, v = fwht_reference(k), fwht_reference(v)
        kp[r], vp[r] = k.to(dtype), v.to(dtype)

    for blk, d0 in zip(c["page_blk"].tolist(), c["page_dst"].tolist()):
        k, v = dequant(blk)
        for t in range(PAGE):
            put(d0 + t, k[:, t], v[:, t])
    info = c["tail_info"].view(-1, 3).tolist()
    for blk, (d0, n, slot) in zip(c["tail_blk"].tolist(), info):
        _, v = dequant(blk)
        for t in range(n):
            put(d0 + t, c["tail_k"][slot, :, t].float(), v[:, t])
    for j, r in enumerate(c["new_dst"].tolist()):
        kp[r], vp[r] = c["k_new"][j], c["v_new"][j]
    return kp, vp


def history_rows(c: dict) -> torch.Tensor:
    """Rows written from the cache (full and partial pages), in order."""
    rows = [d0 + t for d0 in c["page_dst"].tolist() for t in range(PAGE)]
    rows += [d0 + t for d0, n, _ in c["tail_info"].view(-1, 3).tolist() for t in range(n)]
    return torch.tensor(rows, dtype=torch.long)
