"""Shared case of the rotation-benefit tests (CPU oracle and GPU): int4 attention error with and
without the Hadamard rotation, for K and V with outlier channels (reference:
tests/test_cpu.py:369-393)."""
import torch
import torch.nn.functional as F

from kushkash_amd._ops import PAGE


def rotation_errors(make_cache, dev) -> dict:
    """{rot: (decode rel-error, chunk rel-error)} against exact fp32 attention; make_cache(rot)
    builds a 1-layer cache of batch 1, 2 kv heads, 8 q heads, head_dim 128, int4, fp32."""
    g = torch.Generator().manual_seed(1)
    B, H, G, D, n = 1, 2, 4, 128, 4 * PAGE + 7
    K, V = torch.randn(B, H, n, D, generator=g), torch.randn(B, H, n, D, generator=g)
    K[..., [3, 77]] *= 12                                                  # K outlier channels
    V[..., :, 5] += 6 * torch.randn(B, H, n, generator=g)                  # V outlier channel
    q, qc = torch.randn(B, H * G, D, generator=g), torch.randn(B, H * G, 9, D, generator=g)
    kc, vc = torch.randn(B, H, 9, D, generator=g), torch.randn(B, H, 9, D, generator=g)
    exact = F.scaled_dot_product_attention(q[:, :, None], K.repeat_interleave(G, 1),
                                           V.repeat_interleave(G, 1))[:, :, 0]
    Kx, Vx = torch.cat([K, kc], 2), torch.cat([V, vc], 2)
    mask = torch.ones(9, n + 9, dtype=torch.bool).tril(diagonal=n)
    exact_c = F.scaled_dot_product_attention(qc, Kx.repeat_interleave(G, 1), Vx.repeat_interleave(G, 1),
                                             attn_mask=mask)
    err = {}
    for rot in (False, True):
        c = make_cache(rot)
        c.write(0, K.to(dev), V.to(dev))
        d = (c.attend(0, q.to(dev)).cpu() - exact).norm() / exact.norm()
        ch = (c.attend_chunk(0, qc.to(dev), kc.to(dev), vc.to(dev)).cpu() - exact_c).norm() / exact_c.norm()
        hk, _ = c.dequantize(0)
        assert (hk.cpu() - K).abs().max() < 0.6 * K.abs().max()           # dequantize() is in model space
        err[rot] = (float(d), float(ch))
    return err
