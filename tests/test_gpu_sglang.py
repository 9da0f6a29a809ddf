"""The SGLang plugin on the gfx950 kernels (MI355X): the serving sessions of test_sglang.py -- fresh
prompts, mid-page chunks, a shared radix-cache prefix, decodes across page boundaries, padded graph
metadata, multi-request extends -- through KushSGLangBackend with the GPU Ops, and a decode step
captured as a HIP graph (the step's metadata preparation included, as SGLang captures it) replayed
with eager steps in between. Checked against float64 attention over the reference quantization of
the exact tokens (the codes match the kernels' exactly; what remains is the kernels' float
arithmetic and the rounding of the output to the model dtype)."""
import types

import pytest
import torch

from _sglang_world import Layer, Mode, Server, sglang_standins
from test_sglang import serving_session

pytestmark = pytest.mark.gpu

# relative (Frobenius) error bounds of a step's output: fp32 output from fp16 MFMA products with fp32
# accumulation; bf16 adds the output's rounding (2^-9 relative) and the bf16 rounding of rotated tails
BOUND = {torch.float32: 2e-3, torch.bfloat16: 6e-3}


@pytest.fixture(scope="module")
def sg():
    with sglang_standins() as mods:
        yield mods


def _server(sg, monkeypatch, dtype, bits, rot, D=128, **kw):
    monkeypatch.setenv("KUSHKASH_BITS", str(bits))
    monkeypatch.setenv("KUSHKASH_ROTATE", "1" if rot else "0")
    return Server(sg, device="cuda", dtype=dtype, bits=bits, Hq=8, Hk=2, D=D, **kw)


@pytest.mark.parametrize("dtype,bits,rot,mode,D", [
    (torch.bfloat16, 4, True, "packed", 128), (torch.bfloat16, 4, False, "packed", 128),
    (torch.bfloat16, 8, False, "packed", 128), (torch.bfloat16, 8, True, "loop", 128),
    (torch.float32, 4, True, "packed", 128), (torch.float32, 8, False, "loop", 64),
    (torch.bfloat16, 4, True, "packed", 64)])
def test_serving_session_on_the_kernels(sg, monkeypatch, dtype, bits, rot, mode, D):
    monkeypatch.setenv("KUSHKASH_PREFILL", mode)
    w = _server(sg, monkeypatch, dtype, bits, rot, D=D)
    print(f"serving session dtype {dtype} bits {bits} rot {rot} {mode} D {D}", flush=True)
    worst = serving_session(w, torch.Generator().manual_seed(0))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst < BOUND[dtype], worst


def test_small_pack_budget_on_the_kernels(sg, monkeypatch):
    """Several packed groups and the blocked per-request path in one step, on the kernels."""
    w = _server(sg, monkeypatch, torch.bfloat16, 4, True, context=2048, pages=160)
    gen = torch.Generator().manual_seed(3)
    assert w.step([1, 2, 3], [52, 21, 80], False, gen) < BOUND[torch.bfloat16]
    monkeypatch.setenv("KUSHKASH_PACK_MB", "1")            # 1 MiB: 1024 keys of bf16 K + V at Hk 2, D 128
    assert w.step([1, 2, 3], [300, 800, 1100], False, gen) < BOUND[torch.bfloat16]     # 352, 821, 1180 keys
    kinds = [(g.r0, g.r1, g.packed) for g in w.backend.forward_metadata.extend.groups]
    assert kinds == [(0, 1, True), (1, 2, True), (2, 3, False)], kinds
    assert w.step([1, 2, 3], [1, 1, 1], True, gen) < BOUND[torch.bfloat16]


def test_decode_graph_replays(sg, monkeypatch):
    """A padded decode batch captured once (metadata preparation and every layer's forward_decode) and
    replayed for 12 steps, each checked against the reference, with eager decode and extend steps and
    host synchronizations between the replays."""
    dtype = torch.bfloat16
    w = _server(sg, monkeypatch, dtype, 4, True)
    gen = torch.Generator().manual_seed(5)
    A, B, C = 3, 1, 6
    w.step([A, B, C], [75, 31, 130], False, gen)
    w.step([A, B, C], [1, 1, 1], True, gen)                  # eager decode first: kernels loaded
    bs, live = 4, [A, B, C]
    w.backend.init_cuda_graph_state(max_bs=bs, max_num_tokens=bs)
    dev = torch.device("cuda")
    req = torch.zeros(bs, dtype=torch.int64, device=dev)
    lens = torch.ones(bs, dtype=torch.int64, device=dev)
    fb = types.SimpleNamespace(forward_mode=Mode(True), req_pool_indices=req, seq_lens=lens)
    q_in = [torch.zeros(bs, w.Hq * w.D, dtype=dtype, device=dev) for _ in range(w.layers)]
    k_in = [torch.zeros(bs, w.Hk * w.D, dtype=dtype, device=dev) for _ in range(w.layers)]
    v_in = [torch.zeros(bs, w.Hk * w.D, dtype=dtype, device=dev) for _ in range(w.layers)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                           # warm the metadata ops outside the capture
        w.backend.init_forward_metadata_out_graph(fb)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        w.backend.init_forward_metadata_out_graph(fb)
        outs = [w.backend.forward_decode(q_in[i], k_in[i], v_in[i], Layer(i, w.Hq, w.Hk, w.D), fb)
                for i in range(w.layers)]
    for step in range(12):
        before = [w.length[s] for s in live]
        for s in live:
            w.grow(s, 1)
        req.copy_(torch.tensor(live + [0] * (bs - len(live))))
        lens.copy_(torch.tensor([w.length[s] for s in live] + [1] * (bs - len(live))))
        refs = []
        for i in range(w.layers):
            q, k, v = w.inputs(bs, gen)
            q_in[i].copy_(q)
            k_in[i].copy_(k)
            v_in[i].copy_(v)
            refs.append(w.expected(i, live, [1] * len(live), q, k, v, True, before))
        graph.replay()
        torch.cuda.synchronize()
        for i in range(w.layers):
            got = outs[i][:len(live)].double().cpu()
            err = float((got - refs[i]).norm() / refs[i].norm())
            assert err < BOUND[dtype], (step, i, err)
        if step % 4 == 1:                                   # eager work between replays
            assert w.step(live, [1, 1, 1], True, gen) < BOUND[dtype]
        if step % 4 == 3:
            assert w.step([B], [9], False, gen) < BOUND[dtype]
    print(f"graph replays checked; lengths {[w.length[s] for s in live]}", flush=True)
