"""The fused append + decode (kush_append_decode, Ops.append_decode, KushCache.append_attend; needs an
MI355X): the same cache bytes, K tails and outputs as append (pos_offset -1, advance 0) followed by
decode, the reference's two launches (kushkash/_ops.py:66-80, :191-213).

Covered: tokens that complete a page (the page then belongs to a split other than the last one:
160 tokens in 4 splits put page 4 in split 2) and tokens that land mid-page (the tail's split),
sequences of one token, padding rows (seq_lens 0: nothing appended, zero output), split-K merged
in the launch and by the combine kernel, 2 / 4 / 8 waves, int4 / int8, head_dim 64 / 128 / 256,
rotation folded into the kernels, and the fallbacks to the two calls (more than 16 q heads per kv
head, k rows that are not 16-byte aligned)."""
import pytest
import torch

import kushkash_amd as kk
from kushkash_amd._ops import PAGE

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _state(ops, lens, H, D, dtype, seed):
    """A cache of ragged sequences written by the chunk write (lengths before the step's token)."""
    g = torch.Generator().manual_seed(seed)
    S = len(lens)
    pages = -(-(max(lens) + 3) // PAGE)
    cache = torch.zeros(S * pages, H, kk.record_bytes(D, ops.bits), dtype=torch.uint8, device=DEV)
    bt = torch.randperm(S * pages, generator=g, dtype=torch.int32).view(S, pages).to(DEV)
    tail_k = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
    tail_idx = torch.arange(S, dtype=torch.int32, device=DEV)
    n = sum(lens)
    if n:
        k = (torch.randn(n, H, D, generator=g) * 2).to(dtype).to(DEV)
        v = torch.randn(n, H, D, generator=g).to(dtype).to(DEV)
        qsl = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(S)], dtype=torch.int32, device=DEV)
        jobs = [(s, p) for s in range(S) for p in range(-(-lens[s] // PAGE))]
        js = torch.tensor([j[0] for j in jobs], dtype=torch.int32, device=DEV)
        jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32, device=DEV)
        ops.write(k, v, qsl, torch.tensor(lens, dtype=torch.int32, device=DEV), tail_idx, js, jp, cache, bt, tail_k)
    return cache, bt, tail_k, tail_idx


@pytest.mark.parametrize("rot", [False, True])
@pytest.mark.parametrize("ns,waves,merge", [(1, 4, True), (1, 2, True), (1, 8, True), (4, 4, True), (4, 2, False),
                                            (3, 8, True)])
@pytest.mark.parametrize("D,bits,G,dtype", [(128, 4, 7, torch.bfloat16), (128, 8, 4, torch.float16),
                                            (64, 4, 16, torch.bfloat16), (256, 4, 2, torch.float32),
                                            (256, 8, 8, torch.bfloat16)])
def test_fused_equals_append_then_decode(D, bits, G, dtype, ns, waves, merge, rot, monkeypatch):
    import kushkash_amd._ops as ops_mod
    if not merge:
        monkeypatch.setattr(ops_mod, "SYNC_SLOTS", 0)
    ops = kk.Ops(torch.device(DEV), D, bits, G, dtype)
    H = 2
    # before the step: 159 (the token completes page 4 of 5), 0 (first token), 40 (mid-page), 95,
    # 31 (completes page 0), and a padding row (-1: seq_lens stays 0, nothing appended)
    lens = [159, 0, 40, 95, 31, 0]
    pad = 5
    S = len(lens)
    states = [_state(ops, lens, H, D, dtype, seed=D + bits + G) for _ in range(2)]
    g = torch.Generator().manual_seed(7)
    work = [torch.empty(S * H * ns * G * (D + 2), dtype=torch.float32, device=DEV) for _ in range(2)]
    seq_lens = [torch.tensor(lens, dtype=torch.int32, device=DEV) for _ in range(2)]
    for step in range(3):
        k = torch.randn(S, H, D, generator=g).to(dtype).to(DEV)
        v = torch.randn(S, H, D, generator=g).to(dtype).to(DEV)
        q = torch.randn(S, H * G, D, generator=g).to(dtype).to(DEV)
        outs = []
        for i, fused in enumerate((True, False)):
            cache, bt, tail_k, tail_idx = states[i]
            sl = seq_lens[i]
            sl[:pad] += 1                                    # the step's token is counted (vLLM convention)
            out = torch.empty_like(q)
            if fused:
                ops.append_decode(k, v, q, out, cache, bt, sl, tail_idx, tail_k, D ** -0.5, ns, work[i], waves=waves,
                                  rot=rot)
            else:
                ops.append(k, v, sl, tail_idx, cache, bt, tail_k, -1, False, rot=rot)
                ops.decode(q, out, cache, bt, sl, tail_idx, tail_k, D ** -0.5, ns, work[i], waves=waves, rot=rot)
            outs.append(out.float().cpu())
        torch.cuda.synchronize()
        assert torch.equal(states[0][0].cpu(), states[1][0].cpu()), step         # records
        assert torch.equal(states[0][2].cpu(), states[1][2].cpu()), step         # K tails
        assert torch.equal(outs[0][pad], torch.zeros_like(outs[0][pad]))         # padding row
        assert torch.equal(outs[0], outs[1]), step
    assert int(ops._sync.abs().sum()) == 0


@pytest.mark.parametrize("case", ["G > 16", "unaligned k"])
def test_fallbacks_give_the_same_result(case):
    D, bits, dtype, H = 128, 4, torch.bfloat16, 2
    G = 20 if case == "G > 16" else 4
    ops = kk.Ops(torch.device(DEV), D, bits, G, dtype)
    lens = [63, 10]
    S = len(lens)
    states = [_state(ops, lens, H, D, dtype, seed=3) for _ in range(2)]
    g = torch.Generator().manual_seed(8)
    big = torch.randn(S, H * D + 1, generator=g).to(dtype).to(DEV)
    k = big[:, 1:].unflatten(1, (H, D)) if case == "unaligned k" else big[:, :H * D].unflatten(1, (H, D)).contiguous()
    v = torch.randn(S, H, D, generator=g).to(dtype).to(DEV)
    q = torch.randn(S, H * G, D, generator=g).to(dtype).to(DEV)
    outs = []
    for i, fused in enumerate((True, False)):
        cache, bt, tail_k, tail_idx = states[i]
        sl = torch.tensor([n + 1 for n in lens], dtype=torch.int32, device=DEV)
        out = torch.empty_like(q)
        if fused:
            ops.append_decode(k, v, q, out, cache, bt, sl, tail_idx, tail_k, D ** -0.5)
        else:
            ops.append(k, v, sl, tail_idx, cache, bt, tail_k, -1, False)
            ops.decode(q, out, cache, bt, sl, tail_idx, tail_k, D ** -0.5)
        outs.append(out.cpu())
    assert torch.equal(states[0][0].cpu(), states[1][0].cpu())
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("rotate,in_kernels", [(False, False), (True, False), (True, True)])
def test_kushcache_append_attend(rotate, in_kernels):
    """KushCache.append_attend == write (one token) then attend, over 40 steps that cross pages."""
    B, Hq, Hkv, D = 2, 28, 4, 128
    g = torch.Generator().manual_seed(11)
    caches = [kk.KushCache(1, Hkv, Hq, D, batch_size=B, bits=4, device=DEV, dtype=torch.bfloat16, rotate=rotate,
                           rotate_in_kernels=in_kernels) for _ in range(2)]
    K = torch.randn(B, Hkv, 50, D, generator=g).to(torch.bfloat16).to(DEV)
    for c in caches:
        c.write(0, K, K.flip(2))
    for step in range(40):
        k = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        v = torch.randn(B, Hkv, 1, D, generator=g).to(torch.bfloat16).to(DEV)
        q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16).to(DEV)
        a = caches[0].append_attend(0, q, k, v)
        caches[1].write(0, k, v)
        b = caches[1].attend(0, q)
        assert torch.equal(a, b), step
    assert caches[0].length(0) == caches[1].length(0) == 90
    assert torch.equal(caches[0].seq_lens, caches[1].seq_lens)
    assert torch.equal(caches[0].pool, caches[1].pool) and torch.equal(caches[0].tail_k, caches[1].tail_k)
