"""The gfx950 packed-prefill unpack (needs an MI355X): bit-identical to the oracle's CPU kernel
(the reference's, restated) rounded to the output dtype, for every head_dim, bits, dtype and rot,
with rows no entry names left untouched (reference: tests/test_gpu.py:221-240). Also a large
group across all the shape classes a serving step makes (hundreds of shuffled pages, several kv
heads, partial pages of every length, a ragged new chunk), the per-element path for unaligned
rows, index validation before any launch, and the unpack in its use: a packed-prefill group built
from a KushCache, attended per sequence, against attend_chunk."""
import pytest
import torch

import kushkash_amd as kk
from _unpack_fixture import INDEX_NAMES, make_group
from oracle.cpu_ops import OracleOps

pytestmark = pytest.mark.gpu
DEV = "cuda"
BITS_OF = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}


def oracle_unpack(c, D, bits, rot, dtype):
    """The oracle's fp32 kp, vp rounded once to dtype (the kernels round fp32 -> dtype once)."""
    shape = (c["rows"], c["H"], D)
    kp, vp = torch.full(shape, float("nan")), torch.full(shape, float("nan"))
    args = [c[n].float() if n in ("tail_k", "k_new", "v_new") else c[n] for n in INDEX_NAMES]
    OracleOps("cpu", D, bits, 1).unpack(c["records"], *args, kp, vp, rot)
    return kp.to(dtype), vp.to(dtype)


def gpu_unpack(c, D, bits, rot, dtype, k_new=None, v_new=None, kp=None, vp=None):
    shape = (c["rows"], c["H"], D)
    kp = torch.full(shape, float("nan"), dtype=dtype, device=DEV) if kp is None else kp
    vp = torch.full(shape, float("nan"), dtype=dtype, device=DEV) if vp is None else vp
    args = {n: c[n].to(DEV) for n in INDEX_NAMES}
    if k_new is not None:
        args["k_new"], args["v_new"] = k_new, v_new
    kk.Ops(torch.device(DEV), D, bits, 1, dtype).unpack(c["records"].to(DEV), *[args[n] for n in INDEX_NAMES],
                                                        kp, vp, rot)
    return kp.cpu(), vp.cpu()


def assert_same(c, got, want, dtype):
    written = torch.ones(c["rows"], dtype=torch.bool)
    written[torch.tensor(c["gaps"])] = False
    for g, w in zip(got, want):
        a, b = g[written].view(BITS_OF[dtype]), w[written].view(BITS_OF[dtype])
        assert torch.equal(a, b), f"{(a != b).sum().item()} of {a.numel()} values differ from the oracle"
        assert g[~written].isnan().all(), "a row no entry names was written"


@pytest.mark.parametrize("D,bits", [(64, 4), (128, 4), (256, 4), (64, 8), (128, 8), (256, 8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rot", [False, True])
def test_unpack_gpu_matches_oracle(D, bits, dtype, rot):
    c = make_group(D, bits, dtype, seed=D + bits)
    assert_same(c, gpu_unpack(c, D, bits, rot, dtype), oracle_unpack(c, D, bits, rot, dtype), dtype)


@pytest.mark.parametrize("rot", [False, True])
def test_unpack_gpu_large_group(rot):
    """8 kv heads, 300 shuffled full pages, partial pages of 1..31 tokens, 700 new rows in runs."""
    D, bits, dtype = 128, 4, torch.bfloat16
    c = make_group(D, bits, dtype, seed=11, H=8, n_pages=300, tail_tokens=tuple(range(1, 32, 2)),
                   new_runs=(1, 31, 32, 33, 603), slots=24)
    assert_same(c, gpu_unpack(c, D, bits, rot, dtype), oracle_unpack(c, D, bits, rot, dtype), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_unpack_gpu_unaligned_rows(dtype):
    """k_new / v_new rows one element apart from 16-byte alignment, kp / vp starting one element
    into their buffer: the per-element path gives the same bits."""
    D, bits = 128, 8
    c = make_group(D, bits, dtype, seed=5, H=4)
    n, H, rows = c["k_new"].shape[0], c["H"], c["rows"]

    def odd_rows(x):                                   # [n, H, D] with row stride H * D + 1
        buf = torch.empty(n, H * D + 1, dtype=dtype, device=DEV)
        buf[:, :H * D] = x.reshape(n, H * D).to(DEV)
        return buf[:, :H * D].view(n, H, D)

    def offset_out():
        buf = torch.full((rows * H * D + 1,), float("nan"), dtype=dtype, device=DEV)
        return buf[1:].view(rows, H, D)

    k_new, v_new = odd_rows(c["k_new"]), odd_rows(c["v_new"])
    assert k_new.stride(0) == H * D + 1
    got = gpu_unpack(c, D, bits, True, dtype, k_new, v_new, offset_out(), offset_out())
    assert_same(c, got, oracle_unpack(c, D, bits, True, dtype), dtype)


def test_unpack_gpu_validates_indices_before_launch():
    D, bits, dtype = 64, 4, torch.bfloat16
    c = make_group(D, bits, dtype)
    ops = kk.Ops(torch.device(DEV), D, bits, 1, dtype, validate=True)
    shape = (c["rows"], c["H"], D)
    kp = torch.zeros(shape, dtype=dtype, device=DEV)
    args = {n: c[n].to(DEV) for n in INDEX_NAMES}
    args["page_blk"] = args["page_blk"] + c["records"].shape[0]
    with pytest.raises(ValueError, match="page_blk"):
        ops.unpack(c["records"].to(DEV), *[args[n] for n in INDEX_NAMES], kp, kp.clone(), False)
    assert not kp.any()
    empty = torch.zeros(0, dtype=torch.int32, device=DEV)             # nothing to do: no launch
    none = torch.zeros(0, c["H"], D, dtype=dtype, device=DEV)
    ops.unpack(c["records"].to(DEV), empty, empty, empty, empty, args["tail_k"], none, none, empty, kp, kp, False)
    with pytest.raises(ValueError, match="must be torch.bfloat16"):
        ops.unpack(c["records"].to(DEV), *[args[n] if n != "k_new" else args[n].float() for n in INDEX_NAMES],
                   kp, kp.clone(), False)


def test_packed_prefill_matches_attend_chunk():
    """The unpack in its use (the vLLM packed prefill, kushkash/vllm/backend.py:837-856): a group
    built from a KushCache's own block table, records and K tail -- each sequence's history (two
    full pages and a partial one, K from the tail slot) followed by its new chunk -- unpacks to the
    exact dequantization of those records (bit for bit, the fp64 restatement), and attention per
    sequence over its packed rows, causal from the history's end, agrees with attend_chunk over the
    same cache. attend_chunk unpacks its history blocks with the same kernel but rotates them back and
    blocks the keys differently, so the two differ by rounding: max-abs within 2e-2."""
    import torch.nn.functional as F
    from _unpack_fixture import unpack_torch
    from kushkash_amd._ops import PAGE
    B, Hkv, G, D, hist, T = 2, 2, 4, 128, 70, 33
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(7)
    c = kk.KushCache(1, Hkv, Hkv * G, D, batch_size=B, bits=4, device=DEV, dtype=dt, rotate=False)
    c.write(0, torch.randn(B, Hkv, hist, D, generator=g).to(dt).to(DEV),
            torch.randn(B, Hkv, hist, D, generator=g).to(dt).to(DEV))
    q = torch.randn(B, Hkv * G, T, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, T, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, T, D, generator=g).to(dt)
    bt, ti = c.block_table.cpu(), c.tail_idx.cpu()
    full, rem = divmod(hist, PAGE)
    L = hist + T                                                          # packed rows per sequence
    i32 = lambda x: torch.tensor(x, dtype=torch.int32)
    group = dict(records=c.pool[0].cpu(), H=Hkv, rows=B * L, gaps=[],
                 page_blk=i32([int(bt[i, p]) for i in range(B) for p in range(full)]),
                 page_dst=i32([i * L + p * PAGE for i in range(B) for p in range(full)]),
                 tail_blk=i32([int(bt[i, full]) for i in range(B)]),
                 tail_info=i32([x for i in range(B) for x in (i * L + full * PAGE, rem, int(ti[i]))]),
                 tail_k=c.tail_k[0].cpu(), k_new=k.permute(0, 2, 1, 3).reshape(B * T, Hkv, D),
                 v_new=v.permute(0, 2, 1, 3).reshape(B * T, Hkv, D),
                 new_dst=i32([i * L + hist + t for i in range(B) for t in range(T)]))
    kp = torch.zeros(B * L, Hkv, D, dtype=dt, device=DEV)
    vp = torch.zeros_like(kp)
    c.ops.unpack(c.pool[0], *[group[n].to(DEV) for n in INDEX_NAMES], kp, vp, False)
    want_k, want_v = unpack_torch(group, D, 4, False, dt)
    assert torch.equal(kp.cpu().view(torch.int16), want_k.view(torch.int16))
    assert torch.equal(vp.cpu().view(torch.int16), want_v.view(torch.int16))
    keys = kp.view(B, L, Hkv, D).permute(0, 2, 1, 3).float().cpu()
    vals = vp.view(B, L, Hkv, D).permute(0, 2, 1, 3).float().cpu()
    mask = torch.ones(T, L, dtype=torch.bool).tril(hist)                  # query t sees hist + t + 1 rows
    out = F.scaled_dot_product_attention(q.float(), keys, vals, attn_mask=mask, enable_gqa=True)
    ref = c.attend_chunk(0, q.to(DEV), k.to(DEV), v.to(DEV)).float().cpu()
    err = (out - ref).abs().max().item()
    assert err < 2e-2, err


@pytest.mark.parametrize("seed", range(60))
def test_unpack_random_groups(seed):
    """Seeded random groups, bit-identical to the oracle: head dim, bits, dtype, rot, 1-8 kv heads (the
    row-by-row path when a workgroup's tasks are heads of one page, the per-task path otherwise),
    0-40 full pages, 0-6 partial pages of 1-31 tokens, 0-4 runs of new rows, aligned or unaligned
    new rows; rows no entry names stay untouched."""
    import numpy as np
    rng = np.random.default_rng(7000 + seed)
    D, bits = int(rng.choice([64, 128, 256])), int(rng.choice([4, 8]))
    dtype = (torch.float32, torch.bfloat16, torch.float16)[rng.integers(3)]
    rot, H = bool(rng.random() < 0.5), int(rng.integers(1, 9))
    tails = tuple(int(x) for x in rng.integers(1, 32, int(rng.integers(0, 7))))
    runs = tuple(int(x) for x in rng.integers(1, 81, int(rng.integers(0, 5))))
    c = make_group(D, bits, dtype, seed=seed, H=H, n_pages=int(rng.integers(0, 41)), tail_tokens=tails,
                   new_runs=runs, slots=len(tails) + int(rng.integers(1, 4)))
    print(f"seed {seed}: D {D} bits {bits} {dtype} rot {rot} H {H} pages {c['page_blk'].numel()} tails {tails} "
          f"runs {runs}", flush=True)
    k_new = v_new = None
    if rng.random() < 0.3 and c["k_new"].shape[0]:                  # new rows one element off 16-byte alignment
        n = c["k_new"].shape[0]

        def odd_rows(x):
            buf = torch.empty(n, H * D + 1, dtype=dtype, device=DEV)
            buf[:, :H * D] = x.reshape(n, H * D).to(DEV)
            return buf[:, :H * D].view(n, H, D)
        k_new, v_new = odd_rows(c["k_new"]), odd_rows(c["v_new"])
    got = gpu_unpack(c, D, bits, rot, dtype, k_new, v_new)
    assert_same(c, got, oracle_unpack(c, D, bits, rot, dtype), dtype)


@pytest.mark.parametrize("D,bits", [(128, 4), (64, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rot", [False, True])
def test_torch_unpack_equals_the_kernel(D, bits, dtype, rot):
    """KUSHKASH_UNPACK=torch (kushkash_amd._serving.torch_unpack, the serving switch's torch path) gives
    the unpack kernel's bits on the GPU, and leaves the same gap rows untouched."""
    from kushkash_amd._serving import torch_unpack
    c = make_group(D, bits, dtype, seed=3 * D + bits)
    shape = (c["rows"], c["H"], D)
    kp = torch.full(shape, float("nan"), dtype=dtype, device=DEV)
    vp = torch.full(shape, float("nan"), dtype=dtype, device=DEV)
    args = [c[n].to(DEV) for n in INDEX_NAMES]
    torch_unpack(c["records"].to(DEV), *args, kp, vp, D, bits, rot)
    assert_same(c, (kp.cpu(), vp.cpu()), gpu_unpack(c, D, bits, rot, dtype), dtype)
