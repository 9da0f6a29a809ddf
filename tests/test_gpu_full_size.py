"""Decode at the benchmark configurations' full sizes (needs an MI355X), built exactly as bench.py
builds them: the outputs match the reference's own dequant-attention -- fp32 attention over the
records dequantized by the torch reference path (cached_kv, kushkash/_ops.py:295-306; the partial
page with its exact K tail) -- every element within 2e-3 plus its own rounding to the output dtype
(bf16 out, fp32 accumulation: the acceptance bound of the compressed-KV decode).

C2: Qwen2.5-7B layer, int4, 64 x 4096 tokens (the headline line's workload), bf16; and the same in
    fp32, held to a flat 2e-3 (its own rounding is ~1e-7).
C3: Llama-3.1-8B layer, int8, 128 ragged sequences U[256, 8192] with one appended token each and
    the longest-first order, 2 waves; the append and decode in one launch (the bench line's step) and
    in two.
C4: Qwen3-8B layer, int4, 8 x 131,072 tokens, split-K at the policy's count and at 64, 128 and 256
    splits, merged in the launch and by the combine kernel."""
import math

import pytest
import torch
import torch.nn.functional as F

import bench
from _harness import assert_out_close
from kushkash_amd._ops import PAGE, cached_kv

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def reference(q, cache, table, n, tail_k, D, bits):
    """fp32 attention of q [B, Hq, D] over the n cached tokens of every sequence of the batch."""
    k, v = cached_kv(cache, table, n, tail_k, D, bits, torch.float32)
    return F.scaled_dot_product_attention(q[:, :, None].float(), k, v, enable_gqa=True)[:, :, 0]


def check(out, ref, what, dtype=torch.bfloat16):
    assert_out_close(out, ref, dtype, what=what)


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_c2_full_size(dtype):
    a = bench.parse_args(["--pools", "1", "--dtype", dtype])
    w = bench.make_workload(a, DEV)
    ops, D = w["ops"], w["D"]
    ns = ops.splits(w["B"], w["Hkv"], w["pages"])
    out = torch.empty_like(w["q"])
    ops.decode(w["q"], out, w["cache"], w["tables"][0], w["seq_lens"], w["tail_idx"], w["tail_k"],
               1.0 / math.sqrt(D), ns, None, waves=ops.waves(w["B"], w["Hkv"], ns, w["pages"]))
    check(out, reference(w["q"], w["cache"], w["tables"][0], w["N"], w["tail_k"], D, w["bits"]), f"C2 {dtype}",
          ops.dtype)


@pytest.mark.parametrize("fused", [True, False])
def test_c3_full_size(fused):
    from kushkash_amd._ops import Ops
    B, Hq, Hkv, D, bits = 128, 32, 8, 128, 8
    G, dtype = Hq // Hkv, torch.bfloat16
    lens = torch.randint(256, 8193, (B,), generator=torch.Generator().manual_seed(0)).tolist()
    ops = Ops(torch.device(DEV), D, bits, G, dtype)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(0)
    cache, table, tail_k, tail_idx = bench.ragged_cache(ops, lens, 1, Hkv, 6.0, 0.10, gen, DEV)
    k_new = torch.randn(B, Hkv, D, generator=gen, device=DEV).to(dtype)
    v_new = torch.randn(B, Hkv, D, generator=gen, device=DEV).to(dtype)
    q = torch.randn(B, Hq, D, generator=gen, device=DEV).to(dtype)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV) + 1
    ns = ops.splits(B, Hkv, max(lens) // PAGE + 1)
    work = torch.empty(max(1, B * Hkv * ns * G * (D + 2)), dtype=torch.float32, device=DEV)
    order = torch.tensor(sorted(range(B), key=lambda i: -lens[i]), dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    launch = dict(waves=ops.waves(B, Hkv, ns, max(lens) // PAGE + 1), order=order)
    if fused:
        ops.append_decode(k_new, v_new, q, out, cache, table, sl, tail_idx, tail_k, 1.0 / math.sqrt(D), ns, work,
                          **launch)
    else:
        ops.append(k_new, v_new, sl, tail_idx, cache, table, tail_k, pos_offset=-1, advance=False)
        ops.decode(q, out, cache, table, sl, tail_idx, tail_k, 1.0 / math.sqrt(D), ns, work, **launch)
    for i in range(B):                                         # ragged: one sequence at a time
        t = int(tail_idx[i])
        ref = reference(q[i:i + 1], cache, table[i:i + 1], lens[i] + 1, tail_k[t:t + 1], D, bits)
        check(out[i:i + 1], ref, f"C3 sequence {i} ({lens[i] + 1} tokens)")


@pytest.fixture(scope="module")
def c4():
    """The C4 workload as bench.py builds it, and the fp32 reference output (two sequences at a time)."""
    from kushkash_amd._ops import Ops
    B, Hq, Hkv, D, bits, N = 8, 32, 8, 128, 4, 131072
    G, dtype = Hq // Hkv, torch.bfloat16
    ops = Ops(torch.device(DEV), D, bits, G, dtype)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(0)
    cache, table, tail_k, tail_idx = bench.ragged_cache(ops, [N] * B, 0, Hkv, 4.0, 0.05, gen, DEV)
    q = torch.randn(B, Hq, D, generator=gen, device=DEV).to(dtype)
    ref = torch.cat([reference(q[s0:s0 + 2], cache, table[s0:s0 + 2], N, tail_k[s0:s0 + 2], D, bits)
                     for s0 in range(0, B, 2)])
    return dict(ops=ops, cache=cache, table=table, tail_k=tail_k, tail_idx=tail_idx, q=q, ref=ref, B=B, Hkv=Hkv,
                G=G, D=D, N=N, sl=torch.full((B,), N, dtype=torch.int32, device=DEV))


@pytest.mark.parametrize("merge", ["in-launch", "combine"])
@pytest.mark.parametrize("ns", [0, 64, 128, 256])
def test_c4_full_size(c4, ns, merge, monkeypatch):
    """C4 decode with the policy's split count (0) and with the 64-256 splits of the configuration,
    the partials merged inside the launch or by the combine kernel, waves by the policy."""
    import kushkash_amd._ops as ops_mod
    if merge == "combine":
        monkeypatch.setattr(ops_mod, "SYNC_SLOTS", 0)
    ops, B, Hkv, G, D, N = c4["ops"], c4["B"], c4["Hkv"], c4["G"], c4["D"], c4["N"]
    ns = ns or ops.splits(B, Hkv, N // PAGE)
    assert ns > 1
    waves = ops.waves(B, Hkv, ns, N // PAGE)
    print(f"C4 decode ns={ns} merge={merge} waves={waves}", flush=True)
    work = torch.empty(B * Hkv * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    out = torch.empty_like(c4["q"])
    ops.decode(c4["q"], out, c4["cache"], c4["table"], c4["sl"], c4["tail_idx"], c4["tail_k"], 1.0 / math.sqrt(D),
               ns, work, waves=waves)
    check(out, c4["ref"], f"C4 ns={ns} {merge}")
    assert int(ops._sync.abs().sum()) == 0


@pytest.mark.parametrize("ns,waves", [(0, 0), (0, 8), (64, 0), (64, 8)])
def test_c4_repeated_steps_are_bit_identical(c4, ns, waves):
    """The same C4 decode step three times gives the same bits, at the policy's launch shape and with 8
    waves (two per SIMD, which the hardware runs at different rates): every wave count sums a fixed
    set of pages in a fixed order, and the split merge folds the splits in a fixed order (reference:
    gpu.mojo:566-807 assigns pages to warps statically)."""
    ops, B, Hkv, G, D, N = c4["ops"], c4["B"], c4["Hkv"], c4["G"], c4["D"], c4["N"]
    ns = ns or ops.splits(B, Hkv, N // PAGE)
    waves = waves or ops.waves(B, Hkv, ns, N // PAGE)
    work = torch.empty(B * Hkv * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    outs = []
    for _ in range(3):
        out = torch.empty_like(c4["q"])
        ops.decode(c4["q"], out, c4["cache"], c4["table"], c4["sl"], c4["tail_idx"], c4["tail_k"],
                   1.0 / math.sqrt(D), ns, work, waves=waves)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
