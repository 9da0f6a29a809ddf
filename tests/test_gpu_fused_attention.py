"""The prefill attention's fused path (torch's flash-attention kernel on gfx950, bf16 / fp16) against its
fp32 products: log-sum-exp and outputs of single blocks (GQA folded, causal with the queries at the end
of the keys), the varlen form over ragged packed rows, and KushCache.attend_chunk over a quantized
history, within bf16 / fp16 rounding."""
import pytest
import torch

import kushkash_amd as kk
from kushkash_amd import _attention as A

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL = {torch.bfloat16: 8e-3, torch.float16: 2e-3}


def _rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("causal,T,N", [(False, 7, 300), (False, 64, 1000), (True, 33, 33), (True, 40, 500)])
def test_block_lse_matches_products(D, dtype, causal, T, N):
    torch.manual_seed(D + T + N)
    B, Hq, Hk = 2, 8, 2
    q = torch.randn(B, Hq, T, D, device=DEV, dtype=dtype)
    k = torch.randn(B, Hk, N, D, device=DEV, dtype=dtype)
    v = torch.randn(B, Hk, N, D, device=DEV, dtype=dtype)
    fused = A._flash(q, k, v, causal, D ** -0.5)
    if D <= 128:
        assert fused is not None, "the flash-attention kernel refused a supported shape"
    if fused is None:
        pytest.skip("the flash-attention kernel does not take this head size")
    o, lse = fused
    o_ref, lse_ref = A.attn_lse(q, k, v, causal, D ** -0.5)
    assert (lse - lse_ref).abs().max().item() < 2e-3
    assert _rel(o, o_ref) < REL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
def test_ragged_varlen_matches_products(D, dtype):
    torch.manual_seed(D)
    T, N = [5, 64, 1, 200, 17], [5, 300, 1000, 200, 1017]
    Hq, Hk = 8, 2
    q = torch.randn(sum(T), Hq, D, device=DEV, dtype=dtype)
    k = torch.randn(sum(N), Hk, D, device=DEV, dtype=dtype)
    v = torch.randn(sum(N), Hk, D, device=DEV, dtype=dtype)
    qs = [0] + torch.tensor(T).cumsum(0).tolist()
    ks = [0] + torch.tensor(N).cumsum(0).tolist()
    cu = (torch.tensor(qs, dtype=torch.int32, device=DEV), torch.tensor(ks, dtype=torch.int32, device=DEV),
          max(T), max(N))
    fused = A.ragged_attention(q, k, v, qs, ks, D ** -0.5, varlen=cu)
    ref = A.ragged_attention(q, k, v, qs, ks, D ** -0.5)
    assert _rel(fused, ref) < REL[dtype]
    for i in range(len(T)):                                     # per row, so no short row hides in the norm
        a, b = qs[i], qs[i + 1]
        assert _rel(fused[a:b], ref[a:b]) < 2 * REL[dtype], i


@pytest.mark.parametrize("rotate", [False, True])
def test_attend_chunk_fused_matches_products(rotate, monkeypatch):
    torch.manual_seed(5)
    B, Hk, Hq, D, T, hist = 2, 2, 8, 128, 300, 5000 + 13
    c = kk.KushCache(1, Hk, Hq, D, batch_size=B, bits=4, device=DEV, dtype=torch.bfloat16, rotate=rotate)
    k = torch.randn(B, Hk, hist, D, device=DEV, dtype=torch.bfloat16)
    c.write(0, k, k.flip(2))
    q = torch.randn(B, Hq, T, D, device=DEV, dtype=torch.bfloat16)
    kn = torch.randn(B, Hk, T, D, device=DEV, dtype=torch.bfloat16)
    vn = torch.randn(B, Hk, T, D, device=DEV, dtype=torch.bfloat16)
    fused = c.attend_chunk(0, q, kn, vn, block_bytes=1 << 22)            # several history blocks
    monkeypatch.setenv("KUSHKASH_ATTN", "fp32")
    ref = c.attend_chunk(0, q, kn, vn, block_bytes=1 << 22)
    assert _rel(fused, ref) < REL[torch.bfloat16]
