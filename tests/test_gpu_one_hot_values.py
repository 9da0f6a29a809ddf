"""Decode outputs that are the attention weights themselves (needs an MI355X). Value row t of every
sequence is the Walsh-Hadamard transform of the one-hot e_t (t < D; later tokens zero), so with the
in-kernel rotation the cache holds V_t = e_t exactly (int4 and int8 alike) and, without it, the
oracle's record of the same row; either way the unrotated output of q head g is its softmax weight
vector over the first D tokens. A wrong score term of one page then moves that page's weights as a
block, by far more than the 2e-3 bound -- the failure of a one-stream page step whose bias MFMA result
was read too early on one branch path, which random values hid in most sessions. Every launch shape
is covered: one and two page streams (G 7, 16, 20), 2 / 4 / 8 waves, rotated or not, int4 / int8,
fp32 / fp16 / bf16 q, sequences of whole and partial pages (64, 100, 192, 237 tokens)."""
import pytest
import torch

import kushkash_amd as kk
from _harness import assert_out_close
from kushkash_amd._ops import PAGE, pages_touched
from oracle.cpu_ops import OracleOps

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 128
LENS = [64, 100, 192, 237]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rot", [False, True])
@pytest.mark.parametrize("G", [7, 16, 20])
@pytest.mark.parametrize("waves", [2, 4, 8])
def test_one_hot_values_give_the_attention_weights(dtype, bits, rot, G, waves):
    print(f"one-hot values: {dtype} int{bits} rot={rot} G={G} waves={waves}", flush=True)
    g = torch.Generator().manual_seed(bits * 1000 + G * 10 + waves + (500 if rot else 0))
    H, S = 2, len(LENS)
    ops = kk.Ops(torch.device(DEV), D, bits, G, dtype)
    oracle = OracleOps("cpu", D, bits, G)

    def fwht(x):
        y = x.float().clone().reshape(-1, D).contiguous()
        return oracle.fwht(y, y).view(x.shape)

    def canon(x):                       # what the kernels store before quantizing: rotated rows rounded to dtype
        return fwht(x).to(dtype).float() if rot else x.float()

    pages = -(-max(LENS) // PAGE)
    bt = torch.randperm(S * pages, generator=g, dtype=torch.int32).view(S, pages)
    tail_idx = torch.randperm(S, generator=g).to(torch.int32)
    RB = kk.record_bytes(D, bits)
    cache_g = torch.zeros(S * pages, H, RB, dtype=torch.uint8, device=DEV)
    tail_g = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
    cache_o = torch.zeros(S * pages, H, RB, dtype=torch.uint8)
    tail_o = torch.zeros(S, H, PAGE, D)
    n = sum(LENS)
    k = (torch.randn(n, H, D, generator=g) * 2 + torch.linspace(-4, 4, D)).to(dtype)
    t = torch.cat([torch.arange(L) for L in LENS])
    eye = torch.eye(D)[t.clamp(max=D - 1)] * (t < D).float().unsqueeze(1)
    v = (fwht(eye) if rot else eye).unsqueeze(1).expand(n, H, D).to(dtype).contiguous()
    qsl = torch.tensor([0] + torch.tensor(LENS).cumsum(0).tolist(), dtype=torch.int32)
    sl = torch.tensor(LENS, dtype=torch.int32)
    jobs = [(s, p) for s in range(S) for p in pages_touched(0, LENS[s])]
    js = torch.tensor([j[0] for j in jobs], dtype=torch.int32)
    jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32)
    ops.write(k.to(DEV), v.to(DEV), qsl.to(DEV), sl.to(DEV), tail_idx.to(DEV), js.to(DEV), jp.to(DEV), cache_g,
              bt.to(DEV), tail_g, fused=True, rot=rot)
    oracle.write(canon(k).contiguous(), canon(v).contiguous(), qsl, sl, tail_idx, js, jp, cache_o, bt, tail_o)
    torch.cuda.synchronize()
    assert torch.equal(cache_g.cpu(), cache_o), "record bytes differ"
    q = torch.randn(S, H * G, D, generator=g).to(dtype)
    out = torch.empty(S, H * G, D, dtype=dtype, device=DEV)
    ops.decode(q.to(DEV), out, cache_g, bt.to(DEV), sl.to(DEV), tail_idx.to(DEV), tail_g, D ** -0.5, 1, None,
               waves=waves, rot=rot)
    torch.cuda.synchronize()
    want = torch.empty(S, H * G, D)
    oracle.decode(canon(q).contiguous(), want, cache_o, bt, sl, tail_idx, tail_o, D ** -0.5)
    if rot:
        want = fwht(want)
    assert_out_close(out.float().cpu(), want, dtype, what=f"{dtype} int{bits} rot={rot} G={G} waves={waves}")
