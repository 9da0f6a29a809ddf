"""Seeded random sessions against the CPU oracle (needs an MI355X): head dim, bits, dtype, kv heads, q
heads per kv head, batch, ragged chunk writes (starting and ending anywhere in a page, some empty),
token appends, the fused append + decode, k / v row strides (aligned or not), split count, waves,
workgroup order and the in-kernel rotation all drawn per case. Every case checks the record bytes
and K tails byte for byte and the decode output per element (2e-3 plus half an output ulp of each
reference value) against the oracle run on the same inputs. With rotation, the oracle's rows and q
are rotated by the oracle's own Walsh-Hadamard transform (fp32, then rounded to the dtype, as the
kernels round), so the rotated cases do not lean on the GPU's transform either."""
import numpy as np
import pytest
import torch

import kushkash_amd as kk
from _harness import assert_out_close
from kushkash_amd._ops import PAGE, pages_touched
from oracle.cpu_ops import OracleOps

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _draw(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    S = int(rng.integers(1, 7))
    case = dict(D=int(rng.choice([64, 128, 256])), bits=int(rng.choice([4, 8])), dtype=DTYPES[rng.integers(3)],
                H=int(rng.choice([1, 2, 4])), G=int(rng.choice([1, 2, 3, 4, 7, 8, 16, 20])), S=S,
                rot=bool(rng.random() < 0.4), fused=bool(rng.random() < 0.7), pad=int(rng.choice([0, 0, 8, 1])),
                waves=[None, 2, 4, 8][rng.integers(4)], ns=int(rng.choice([1, 1, 2, 4, 16])),
                order=bool(rng.random() < 0.5), fused_step=bool(rng.random() < 0.5))
    # 1-3 chunks per sequence (sizes 0-130), then 0-40 one-token appends of the whole batch
    case["chunks"] = [[int(x) if rng.random() > 0.15 else 0 for x in rng.integers(1, 131, S)]
                      for _ in range(int(rng.integers(1, 4)))]
    case["appends"] = int(rng.choice([0, 1, 2, 9, 40]))
    case["data_seed"] = int(rng.integers(1 << 30))
    return case


def _rows(x: torch.Tensor, pad: int) -> torch.Tensor:
    """x [n, H, D] on the GPU as rows of stride H * D + pad (pad 1: rows not 16-byte aligned)."""
    n, H, D = x.shape
    big = torch.zeros(n, H * D + pad, dtype=x.dtype, device=DEV)
    big[:, :H * D] = x.reshape(n, H * D).to(DEV)
    return big[:, :H * D].unflatten(1, (H, D))


@pytest.mark.parametrize("seed", range(160))
def test_random_session_matches_oracle(seed):
    c = _draw(seed)
    D, bits, dtype, H, G, S = c["D"], c["bits"], c["dtype"], c["H"], c["G"], c["S"]
    print(f"seed {seed}: {c}", flush=True)
    g = torch.Generator().manual_seed(c["data_seed"])
    ops = kk.Ops(torch.device(DEV), D, bits, G, dtype)
    oracle = OracleOps("cpu", D, bits, G)

    def canon(x):                       # what the kernels store before quantizing: rotated rows rounded to dtype
        if not c["rot"]:
            return x.float()
        y = x.float().reshape(-1, D).contiguous()
        return oracle.fwht(y, y).view(x.shape).to(dtype).float()

    total = [sum(ch[s] for ch in c["chunks"]) + c["appends"] for s in range(S)]
    pages = max(1, -(-max(total) // PAGE))
    RB = kk.record_bytes(D, bits)
    bt = torch.randperm(S * pages, generator=g, dtype=torch.int32).view(S, pages)
    tail_idx = torch.randperm(S, generator=g).to(torch.int32)           # tail slots permuted
    cache_g = torch.zeros(S * pages, H, RB, dtype=torch.uint8, device=DEV)
    tail_g = torch.zeros(S, H, PAGE, D, dtype=dtype, device=DEV)
    cache_o = torch.zeros(S * pages, H, RB, dtype=torch.uint8)
    tail_o = torch.zeros(S, H, PAGE, D)
    bt_g, ti_g = bt.to(DEV), tail_idx.to(DEV)
    offset = torch.linspace(-4, 4, D)
    lens = [0] * S
    for chunk in c["chunks"]:
        n = sum(chunk)
        if n == 0:
            continue
        k = (torch.randn(n, H, D, generator=g) * 2 + offset).to(dtype)
        v = torch.randn(n, H, D, generator=g).to(dtype)
        new = [lens[s] + chunk[s] for s in range(S)]
        qsl = torch.tensor([0] + list(np.cumsum(chunk)), dtype=torch.int32)
        jobs = [(s, p) for s in range(S) for p in pages_touched(lens[s], new[s])]
        js = torch.tensor([j[0] for j in jobs], dtype=torch.int32)
        jp = torch.tensor([j[1] for j in jobs], dtype=torch.int32)
        sl = torch.tensor(new, dtype=torch.int32)
        ops.write(_rows(k, c["pad"]), _rows(v, c["pad"]), qsl.to(DEV), sl.to(DEV), ti_g, js.to(DEV), jp.to(DEV),
                  cache_g, bt_g, tail_g, fused=c["fused"], rot=c["rot"])
        oracle.write(canon(k).contiguous(), canon(v).contiguous(), qsl, sl, tail_idx, js, jp, cache_o, bt, tail_o)
        lens = new
    q = torch.randn(S, H * G, D, generator=g).to(dtype)
    scale = D ** -0.5
    ns, waves = c["ns"], c["waves"]
    work = torch.empty(S * H * ns * G * (D + 2), dtype=torch.float32, device=DEV)
    order = torch.randperm(S, generator=g).to(torch.int32).to(DEV) if c["order"] else None
    out = torch.empty(S, H * G, D, dtype=dtype, device=DEV)
    for step in range(c["appends"]):
        ka = torch.randn(S, H, D, generator=g).to(dtype)
        va = torch.randn(S, H, D, generator=g).to(dtype)
        lens = [n + 1 for n in lens]
        sl = torch.tensor(lens, dtype=torch.int32)
        last = step == c["appends"] - 1
        if last and c["fused_step"]:                 # the decode step's append inside the decode launch
            ops.append_decode(_rows(ka, c["pad"]), _rows(va, c["pad"]), q.to(DEV), out, cache_g, bt_g, sl.to(DEV),
                              ti_g, tail_g, scale, ns, work, waves=waves, order=order, rot=c["rot"])
        else:
            ops.append(_rows(ka, c["pad"]), _rows(va, c["pad"]), sl.to(DEV), ti_g, cache_g, bt_g, tail_g, -1, False,
                       rot=c["rot"])
        oracle.append(canon(ka).contiguous(), canon(va).contiguous(), sl, tail_idx, cache_o, bt, tail_o, -1, False)
    if not (c["appends"] and c["fused_step"]):
        ops.decode(q.to(DEV), out, cache_g, bt_g, torch.tensor(lens, dtype=torch.int32, device=DEV), ti_g, tail_g,
                   scale, ns, work, waves=waves, order=order, rot=c["rot"])
    torch.cuda.synchronize()
    got_cache, got_tail = cache_g.cpu(), tail_g.float().cpu()
    bad = (got_cache != cache_o).sum().item()
    assert bad == 0, f"{bad} record bytes differ"
    for s in range(S):                                   # the rows the tails hold (older rows are stale by design)
        r = lens[s] % PAGE
        assert torch.equal(got_tail[tail_idx[s], :, :r], tail_o[tail_idx[s], :, :r]), f"sequence {s}: K tail differs"
    want = torch.empty(S, H * G, D)
    oracle.decode(canon(q).contiguous(), want, cache_o, bt, torch.tensor(lens, dtype=torch.int32), tail_idx, tail_o,
                  scale)
    if c["rot"]:
        want = oracle.fwht(want.reshape(-1, D).contiguous()).view(want.shape)
    assert_out_close(out.float().cpu(), want, dtype, what=f"seed {seed}")
