"""The Walsh-Hadamard rotation folded into the write, append and decode kernels (rot = 1; needs an
MI355X). No reference counterpart: the reference rotates with a GEMM around its kernels
(kushkash/_ops.py:489-518) and exposes the canonical FWHT as Ops.fwht (_ops.py:104-126).

- A rotated write / append stores exactly the bytes of Ops.fwht on the rows followed by an unrotated
  write / append: records and K tails bit-exact, over ragged chunks that start and end mid-page
  (tail rows read back, partial pages stashed), one launch and two, then appends.
- A rotated decode equals attention of the rotated q (rounded to the dtype, as Ops.fwht) over the
  stored records, rotated back in fp32: checked against the CPU oracle's decode, rotated back by the
  oracle's FWHT, within the decode tolerance (max-abs 2e-3 plus half an ulp of the output dtype), with
  split-K merged in the launch and by the combine kernel, tails and empty sequences.
- KushCache(rotate_in_kernels=True) attends like fp32 attention over its own dequantized, rotated-back
  contents, in decode and in attend_chunk, and dequantize() undoes its rotation exactly."""
import pytest
import torch
import torch.nn.functional as F

import kushkash_amd as kk
from _harness import assert_out_close, half_ulp, out_bound
from kushkash_amd._ops import PAGE
from oracle.cpu_ops import OracleOps

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _fwht_rows(ops, x):
    """Ops.fwht over the last dim of any [..., D] tensor in the kernel dtype."""
    return ops.fwht(x.reshape(-1, x.shape[-1]).contiguous()).view(x.shape)


def _ragged_writes(ops, S, H, D, dtype, rot, fused, seed):
    """Two ragged chunks per sequence (lengths 20/40/64 then 50/75/94: mid-page starts, completed
    pages that read the tail, partial pages left) and two appends at seq_lens - 1; rot: in the
    kernels, else the rows are rotated by Ops.fwht first. Returns the records and the K tails."""
    g = torch.Generator().manual_seed(seed)
    pages = 4
    cache = torch.zeros(S * pages, H, kk.record_bytes(D, ops.bits), dtype=torch.uint8, device=DEV)
    bt = torch.randperm(S * pages, generator=g, dtype=torch.int32).view(S, pages).to(DEV)
    tail_k = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
    tail_idx = torch.arange(S, dtype=torch.int32, device=DEV)
    lens0, lens1 = [20, 40, 64][:S], [50, 75, 94][:S]
    T = max(lens1)
    kf = (torch.randn(S * T, H, D, generator=g) * 2 + torch.linspace(-3, 3, D)).to(dtype).to(DEV)
    vf = torch.randn(S * T, H, D, generator=g).to(dtype).to(DEV)
    prep = (lambda x: x) if rot else (lambda x: _fwht_rows(ops, x))
    done = [0] * S
    for lens in (lens0, lens1):
        n_new = [lens[s] - done[s] for s in range(S)]
        rows = torch.cat([torch.arange(s * T + done[s], s * T + lens[s]) for s in range(S)]).to(DEV)
        qsl = torch.tensor([0] + [sum(n_new[:i + 1]) for i in range(S)], dtype=torch.int32, device=DEV)
        jobs = [(s, p) for s in range(S) for p in range(done[s] // PAGE, -(-lens[s] // PAGE))]
        js = torch.tensor([j[0] for j in jobs], dtype=torch.int32, device=DEV)
        jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32, device=DEV)
        sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
        ops.write(prep(kf[rows]), prep(vf[rows]), qsl, sl, tail_idx, js, jp, cache, bt, tail_k, fused=fused, rot=rot)
        done = list(lens)
    for step in range(2):
        sl = torch.tensor([n + 1 + step for n in lens1], dtype=torch.int32, device=DEV)
        ka = torch.randn(S, H, D, generator=g).to(dtype).to(DEV)
        va = torch.randn(S, H, D, generator=g).to(dtype).to(DEV)
        ops.append(prep(ka), prep(va), sl, tail_idx, cache, bt, tail_k, pos_offset=-1, advance=False, rot=rot)
    torch.cuda.synchronize()
    return cache.cpu(), tail_k.cpu()


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("D,bits,dtype", [(128, 4, torch.bfloat16), (128, 8, torch.float16), (64, 4, torch.float32),
                                          (256, 4, torch.bfloat16), (256, 8, torch.float32)])
def test_rotated_write_is_fwht_then_write(D, bits, dtype, fused):
    ops = kk.Ops(torch.device(DEV), D, bits, 1, dtype)
    S, H = 3, 2
    c_rot, t_rot = _ragged_writes(ops, S, H, D, dtype, True, fused, seed=D + bits)
    c_ref, t_ref = _ragged_writes(ops, S, H, D, dtype, False, fused, seed=D + bits)
    assert torch.equal(c_rot, c_ref)
    assert torch.equal(t_rot, t_ref)


def _oracle_rotated_decode(cache, bt, lens, tail_idx, tail_k, q_rot, D, bits, G, scale):
    """fp32 oracle decode of the (already rotated) q over the records, rotated back by the oracle's FWHT."""
    o = OracleOps("cpu", D, bits, G)
    want = torch.empty(q_rot.shape)
    o.decode(q_rot.float().cpu().contiguous(), want, cache.cpu(), bt.cpu().contiguous(), lens.cpu(), tail_idx.cpu(),
             tail_k.float().cpu(), scale)
    return o.fwht(want.reshape(-1, D).contiguous()).view(want.shape)


@pytest.mark.parametrize("fused_merge", [True, False])
@pytest.mark.parametrize("ns,waves", [(1, 4), (1, 2), (1, 8), (3, 4), (4, 8)])
@pytest.mark.parametrize("D,bits,G,dtype", [(128, 4, 7, torch.bfloat16), (128, 8, 4, torch.float16),
                                            (64, 4, 20, torch.bfloat16), (256, 4, 2, torch.float32)])
def test_rotated_decode_matches_oracle(D, bits, G, dtype, ns, waves, fused_merge, monkeypatch):
    import kushkash_amd._ops as ops_mod
    if not fused_merge:
        if ns == 1:
            pytest.skip("no split partials to combine")
        monkeypatch.setattr(ops_mod, "SYNC_SLOTS", 0)
    torch.manual_seed(D * G + bits)
    lens = [0, 31, 32, 5 * PAGE + 9, 12 * PAGE]
    S, H = len(lens), 2
    ops = kk.Ops(torch.device(DEV), D, bits, G, dtype)
    pages = -(-max(lens) // PAGE)
    cache = torch.zeros(S * pages, H, kk.record_bytes(D, bits), dtype=torch.uint8, device=DEV)
    bt = torch.randperm(S * pages, dtype=torch.int32).view(S, pages).to(DEV)
    tail_k = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
    tail_idx = torch.arange(S, dtype=torch.int32, device=DEV)
    n = sum(lens)
    k = (torch.randn(n, H, D, device=DEV) * 2).to(dtype)
    v = torch.randn(n, H, D, device=DEV).to(dtype)
    qsl = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(S)], dtype=torch.int32, device=DEV)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=DEV)
    jobs = [(s, p) for s in range(S) for p in range(-(-lens[s] // PAGE))]
    js = torch.tensor([j[0] for j in jobs], dtype=torch.int32, device=DEV)
    jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32, device=DEV)
    ops.write(k, v, qsl, seq_lens, tail_idx, js, jp, cache, bt, tail_k, rot=True)
    q = torch.randn(S, H * G, D, device=DEV).to(dtype)
    work = torch.empty(S * H * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    out = torch.empty_like(q)
    for call in range(2):                            # twice: the split counters reset themselves
        ops.decode(q, out, cache, bt, seq_lens, tail_idx, tail_k, D ** -0.5, ns, work, waves=waves, rot=True)
    q_rot = _fwht_rows(ops, q)                       # the q the kernel attends with (rounded to dtype)
    want = _oracle_rotated_decode(cache, bt, seq_lens, tail_idx, tail_k, q_rot, D, bits, G, D ** -0.5)
    got = out.float().cpu()
    assert torch.equal(got[0], torch.zeros_like(got[0]))                       # empty sequence
    assert_out_close(got, want, dtype)
    assert int(ops._sync.abs().sum()) == 0


@pytest.mark.parametrize("bits,dtype", [(4, torch.bfloat16), (4, torch.float16), (8, torch.bfloat16)])
def test_kushcache_rotate_in_kernels(bits, dtype):
    B, Hq, Hkv, D, N, T = 2, 8, 2, 128, 333, 45
    g = torch.Generator().manual_seed(bits)
    K = torch.randn(B, Hkv, N, D, generator=g).to(dtype).to(DEV)
    V = torch.randn(B, Hkv, N, D, generator=g).to(dtype).to(DEV)
    c = kk.KushCache(1, Hkv, Hq, D, batch_size=B, bits=bits, device=DEV, dtype=dtype, rotate=True,
                     rotate_in_kernels=True)
    assert c.krot
    c.write(0, K[:, :, :200], V[:, :, :200])
    for t in range(200, N):
        c.write(0, K[:, :, t:t + 1], V[:, :, t:t + 1])
    hk, hv = c.dequantize(0)                         # unrotated view of the cache's contents
    # the partial page's K is exact: dequantize() rotates the tail back to the input
    r = N % PAGE
    assert (hk[:, :, N - r:].float() - K[:, :, N - r:].float()).abs().max().item() <= 4 * half_ulp(8.0, dtype)
    q = torch.randn(B, Hq, D, generator=g).to(dtype).to(DEV)
    out = c.attend(0, q).float()
    ref = F.scaled_dot_product_attention(q[:, :, None].float(), hk.float().repeat_interleave(Hq // Hkv, 1),
                                         hv.float().repeat_interleave(Hq // Hkv, 1), scale=c.scale)[:, :, 0]
    # q is rotated and rounded to dtype in the kernel, and dequantize() rounds its rotation of the
    # cache back to dtype: errors spread over every dim by a rotation (at the largest |ref|, plus the
    # keys' rounding as a second 2e-3), then the output's one rounding per element
    bound = out_bound(ref, dtype, base=4e-3) + 2 * half_ulp(float(ref.abs().max()), dtype)
    assert bool(((out - ref).abs() <= bound).all()), (out - ref).abs().max().item()
    qc = torch.randn(B, Hq, T, D, generator=g).to(dtype).to(DEV)
    kc = torch.randn(B, Hkv, T, D, generator=g).to(dtype).to(DEV)
    vc = torch.randn(B, Hkv, T, D, generator=g).to(dtype).to(DEV)
    oc = c.attend_chunk(0, qc, kc, vc).float()
    Kf = torch.cat([hk, kc], 2).float().repeat_interleave(Hq // Hkv, 1)
    Vf = torch.cat([hv, vc], 2).float().repeat_interleave(Hq // Hkv, 1)
    mask = torch.ones(T, N + T, dtype=torch.bool, device=DEV).tril(diagonal=N)
    rc = F.scaled_dot_product_attention(qc.float(), Kf, Vf, attn_mask=mask, scale=c.scale)
    assert (oc - rc).abs().max().item() <= 1e-2
