"""The KushCache API end to end on the GPU with the Hadamard rotation on (needs an MI355X).

test_c1_rotated_cache: the reference's CPU-runnable configuration (batch 1, 8 q / 2 kv heads,
head_dim 128, 512 cached tokens, int4 -- rotation on by default -- bf16 K, V, q ~ N(0, 1) from
seed 0): pack the context, then one attend. The reference checks attend against attention over
the cache's own dequantized keys and values (tests/test_cpu.py:79-96); here that reference runs in
fp32 on the CPU. Two checks: the decode kernel itself, on the rotated q the cache hands it, against
the oracle over the same records (2e-3 plus the output's one rounding, per element); and the API
end to end, where q goes in and the output comes back through bf16 rotation GEMMs (cache.py:174-183):
there the rounding of q and of the kernel's output happen before a rotation that mixes every dim, so
those two count at the largest element, and only the final rounding at each element's own size.

test_attend_chunk_over_history: a chunk of new queries over the cached history plus the chunk
itself, causal (cache.py:185-201), against fp32 attention over [dequantized history | chunk].

The reference's rotation tests on the GPU: rotate() rounds once (tests/test_gpu.py:65-84), a
rotated cache attends like the CPU one (:87-97), and rotation lowers the int4 attention error
(tests/test_cpu.py:369-393)."""
import pytest
import torch
import torch.nn.functional as F

import kushkash_amd as kk
from _harness import assert_out_close, half_ulp, out_bound

pytestmark = pytest.mark.gpu
DEV = "cuda"
def _mixed_bound(ref: torch.Tensor, mixed: int) -> torch.Tensor:
    """Per element: 2e-3 plus the final bf16 rounding at the element's own size, plus `mixed` bf16
    roundings taken before a rotation (which spreads an error of one dim over all dims) at the
    largest |ref|."""
    return out_bound(ref, torch.bfloat16) + mixed * half_ulp(float(ref.abs().max()), torch.bfloat16)


def test_c1_rotated_cache():
    from kushkash_amd._ops import rotate
    from oracle.cpu_ops import OracleOps
    B, Hq, Hkv, D, N = 1, 8, 2, 128, 512
    g = torch.Generator().manual_seed(0)
    K = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16)
    V = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    c = kk.KushCache(1, Hkv, Hq, D, batch_size=B, bits=4, device=DEV, dtype=torch.bfloat16)
    assert c.rot is not None                                           # auto: on for int4
    c.write(0, K.to(DEV), V.to(DEV))
    out = c.attend(0, q.to(DEV)).float().cpu()

    # the kernel on the rotated q, against the oracle over the same records
    q_rot = rotate(q.to(DEV), c.rot, torch.bfloat16).contiguous()
    o_rot = torch.empty_like(q_rot)
    c.ops.decode(q_rot, o_rot, c.pool[0], c.block_table, c.seq_lens[0], c.tail_idx, c.tail_k[0], c.scale)
    want = torch.empty(q_rot.shape)
    OracleOps("cpu", D, 4, Hq // Hkv).decode(q_rot.float().cpu(), want, c.pool[0].cpu(), c.block_table.cpu(),
                                            c.seq_lens[0].cpu(), c.tail_idx.cpu(), c.tail_k[0].float().cpu(), c.scale)
    assert_out_close(o_rot, want, torch.bfloat16, what="C1 kernel vs oracle")

    # end to end through the API, against fp32 attention over the cache's own dequantization
    hk, hv = c.dequantize(0)
    ref = F.scaled_dot_product_attention(q[:, :, None].float(), hk.float().cpu(), hv.float().cpu(),
                                         enable_gqa=True)[:, :, 0]
    err = (out - ref).abs()
    bound = _mixed_bound(ref, 2)
    assert bool((err <= bound).all()), (err.max().item(), (err - bound).max().item())
    rel = ((out - ref).norm() / ref.norm()).item()
    assert rel < 2e-2, rel


@pytest.mark.parametrize("n_hist,T", [(0, 40), (100, 33), (512, 64)])
def test_attend_chunk_over_history(n_hist, T):
    B, Hq, Hkv, D = 2, 8, 2, 128
    g = torch.Generator().manual_seed(n_hist + T)
    c = kk.KushCache(1, Hkv, Hq, D, batch_size=B, bits=4, device=DEV, dtype=torch.bfloat16)
    if n_hist:
        c.write(0, torch.randn(B, Hkv, n_hist, D, generator=g).to(torch.bfloat16).to(DEV),
                torch.randn(B, Hkv, n_hist, D, generator=g).to(torch.bfloat16).to(DEV))
    q = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, D, generator=g).to(torch.bfloat16)
    out = c.attend_chunk(0, q.to(DEV), k.to(DEV), v.to(DEV)).float().cpu()
    if n_hist:
        hk, hv = c.dequantize(0)
        keys, vals = torch.cat([hk.float().cpu(), k.float()], 2), torch.cat([hv.float().cpu(), v.float()], 2)
    else:
        keys, vals = k.float(), v.float()
    n = keys.shape[2]
    mask = torch.ones(T, n, dtype=torch.bool).tril(n - T)              # query t sees n - T + t + 1 keys
    ref = F.scaled_dot_product_attention(q.float(), keys, vals, attn_mask=mask, enable_gqa=True)
    err = (out - ref).abs()
    # q, k, v rotated and rounded, the output rotated back and rounded (cache.py:185-201)
    assert bool((err <= _mixed_bound(ref, 2)).all()), err.max().item()


def test_rotate_rounds_once_gpu():
    """rotate() on the GPU (one torch GEMM with the +-1 matrix and alpha 1/sqrt(D), fp32
    accumulation): within one rounding of the exact product for every dtype and head_dim, and the
    out= form gives the same bits (tests/test_gpu.py:65-84)."""
    from kushkash_amd._ops import hadamard, rotate
    unit = {torch.float32: 2.0 ** -24, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}
    for dt, u in unit.items():
        for D in (64, 128, 256):
            h = hadamard(D, DEV)
            x = torch.randn(6, 8, D, device=DEV).to(dt)[:, ::2]
            y = rotate(x, h)
            ref = x.double() @ h.double()
            tol = u * ref.abs() + 1e-5
            assert y.dtype == dt and bool(((y.double() - ref).abs() <= tol).all()), (dt, D)
            buf = torch.full((8, 4, D), float("nan"), device=DEV, dtype=dt)
            rotate(x, h, out=buf[:6])
            assert torch.equal(buf[:6], y) and bool(buf[6:].isnan().all()), (dt, D)


def test_rotated_cache_gpu_matches_oracle():
    """Rotation on, fp32: GPU and CPU-oracle caches attend alike (pages may differ in rare rounding
    flips of the rotated inputs, the outputs must not; tests/test_gpu.py:87-97)."""
    from _harness import oracle_cache
    torch.manual_seed(0)
    B, H, G, D, T = 2, 2, 4, 128, 3 * 32 + 5
    K, V, q = torch.randn(B, H, T, D) * 2, torch.randn(B, H, T, D), torch.randn(B, H * G, D)
    K[..., 1] += 50
    outs = []
    cpu = oracle_cache(1, H, H * G, D, batch_size=B, bits=4, rotate=True)
    cpu.write(0, K, V)
    outs.append(cpu.attend(0, q))
    gpu = kk.KushCache(1, H, H * G, D, batch_size=B, bits=4, device=DEV, dtype=torch.float32, rotate=True)
    gpu.write(0, K.to(DEV), V.to(DEV))
    outs.append(gpu.attend(0, q.to(DEV)).cpu())
    assert (outs[0] - outs[1]).norm() / outs[0].norm() < 3e-3


def test_rotation_lowers_attention_error_gpu():
    """With outlier channels in K and V, decode and chunk attention over the int4 cache land closer
    to exact attention when the cache rotates (tests/test_cpu.py:369-393), on the GPU path."""
    from _rotation_case import rotation_errors
    err = rotation_errors(lambda rot: kk.KushCache(1, 2, 8, 128, batch_size=1, bits=4, device=DEV,
                                                   dtype=torch.float32, rotate=rot), DEV)
    assert err[True][0] < 0.9 * err[False][0] and err[True][1] < 0.9 * err[False][1], err


def test_attend_chunk_memory_is_bounded():
    """A 1,024-token prefill chunk over 131,072 cached tokens (Qwen3-8B width: 32 q / 8 kv heads, D 128,
    int4, bf16, batch 1): attend_chunk allocates at most 1 GB beyond the cache while it runs (the score
    matrix of the whole history alone would be 17 GB in fp32), and its output matches the torch
    reference path over the same records (history_attention: torch dequantization, key blocks merged by
    log-sum-exp) -- both attend over the same bf16 K / V values, so only fp32 summation order differs."""
    from kushkash_amd._ops import history_attention
    B, Hq, Hkv, D, N, T = 1, 32, 8, 128, 131072, 1024
    g = torch.Generator(device=DEV)
    g.manual_seed(11)
    c = kk.KushCache(1, Hkv, Hq, D, batch_size=B, bits=4, device=DEV, dtype=torch.bfloat16, rotate=False,
                     max_length=N + T)
    for t0 in range(0, N, 16384):
        c.write(0, torch.randn(B, Hkv, 16384, D, generator=g, device=DEV).to(torch.bfloat16),
                torch.randn(B, Hkv, 16384, D, generator=g, device=DEV).to(torch.bfloat16))
    q = torch.randn(B, Hq, T, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, Hkv, T, D, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B, Hkv, T, D, generator=g, device=DEV).to(torch.bfloat16)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = c.attend_chunk(0, q, k, v)
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated() - base
    assert extra <= 1 << 30, f"attend_chunk took {extra / 2**20:.0f} MiB beyond the cache"
    ref = history_attention(q, k, v, c.pool[0], c.block_table, N, c.tail_k[0], D, 4, c.scale)
    assert_out_close(out, ref.float(), torch.bfloat16, base=1e-3, roundings=2, what="attend_chunk vs the torch path")
