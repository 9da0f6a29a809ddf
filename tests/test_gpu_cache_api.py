"""The KushCache API end to end on the GPU with the Hadamard rotation on (needs an MI355X).

test_c1_rotated_cache: the reference's CPU-runnable configuration (batch 1, 8 q / 2 kv heads,
head_dim 128, 512 cached tokens, int4 -- rotation on by default -- bf16 K, V, q ~ N(0, 1) from
seed 0): pack the context, then one attend. The reference checks attend against attention over
the cache's own dequantized keys and values (tests/test_cpu.py:79-96); here that reference runs in
fp32 on the CPU. With rotation, q goes in and the output comes back through bf16 GEMMs
(cache.py:174-183), so the bound is the decode tolerance plus three bf16 roundings at the output's
magnitude.

test_attend_chunk_over_history: a chunk of new queries over the cached history plus the chunk
itself, causal (cache.py:185-201), against fp32 attention over [dequantized history | chunk]."""
import pytest
import torch
import torch.nn.functional as F

import kushkash_amd as kk

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16_HALF_ULP = 2.0 ** -9


def _bound(ref: torch.Tensor, roundings: int) -> float:
    return 2e-3 + roundings * BF16_HALF_ULP * float(ref.abs().max())


def test_c1_rotated_cache():
    B, Hq, Hkv, D, N = 1, 8, 2, 128, 512
    g = torch.Generator().manual_seed(0)
    K = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16)
    V = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    c = kk.KushCache(1, Hkv, Hq, D, batch_size=B, bits=4, device=DEV, dtype=torch.bfloat16)
    assert c.rot is not None                                           # auto: on for int4
    c.write(0, K.to(DEV), V.to(DEV))
    out = c.attend(0, q.to(DEV)).float().cpu()
    hk, hv = c.dequantize(0)
    ref = F.scaled_dot_product_attention(q[:, :, None].float(), hk.float().cpu(), hv.float().cpu(),
                                         enable_gqa=True)[:, :, 0]
    err = (out - ref).abs().max().item()
    assert err <= _bound(ref, 3), err
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
    err = (out - ref).abs().max().item()
    assert err <= _bound(ref, 3), err
