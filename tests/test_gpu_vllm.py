"""The vLLM plugin on the gfx950 kernels (MI355X): the serving sessions of test_vllm.py through the
metadata builder and KushAttentionImpl with the GPU Ops, and uniform single-token decode steps captured
as one HIP graph the way vLLM captures them (metadata built outside the graph into persistent
buffers, a padding row of length 0), replayed with eager steps in between. Checked against float64
attention over the reference quantization of the exact tokens."""
import types

import numpy as np
import pytest
import torch

from _vllm_world import CommonAttentionMetadata, Engine, vllm_standins
from kushkash_amd._ops import PAGE
from test_vllm import serving_session

pytestmark = pytest.mark.gpu
BOUND = {torch.float32: 2e-3, torch.bfloat16: 6e-3}      # relative (Frobenius), as the SGLang GPU tests


@pytest.fixture(scope="module")
def kb():
    with vllm_standins() as backend:
        yield backend


def _engine(kb, monkeypatch, dtype, bits, rot, D=128, **kw):
    monkeypatch.setenv("KUSHKASH_BITS", str(bits))
    monkeypatch.setenv("KUSHKASH_ROTATE", "1" if rot else "0")
    return Engine(kb, device="cuda", dtype=dtype, bits=bits, Hq=8, Hk=2, D=D, **kw)


@pytest.mark.parametrize("dtype,bits,rot,mode,D", [
    (torch.bfloat16, 4, True, "packed", 128), (torch.bfloat16, 4, False, "packed", 128),
    (torch.bfloat16, 8, False, "loop", 128), (torch.float16, 8, True, "packed", 64),
    (torch.bfloat16, 4, True, "packed", 256)])
def test_serving_session_on_the_kernels(kb, monkeypatch, dtype, bits, rot, mode, D):
    monkeypatch.setenv("KUSHKASH_PREFILL", mode)
    w = _engine(kb, monkeypatch, dtype, bits, rot, D=D)
    print(f"vLLM session dtype {dtype} bits {bits} rot {rot} {mode} D {D}", flush=True)
    worst = serving_session(w, torch.Generator().manual_seed(0))
    print(f"worst relative error {worst:.3e}", flush=True)
    assert worst < BOUND[torch.bfloat16 if dtype == torch.float16 else dtype], worst


def test_full_graph_decode_replays(kb, monkeypatch):
    dtype = torch.bfloat16
    w = _engine(kb, monkeypatch, dtype, 4, True)
    gen = torch.Generator().manual_seed(9)
    live = [0, 1, 2]
    for req, slot in zip(live, (4, 1, 6)):
        w.admit(req, slot)
    assert w.step([(0, 75), (1, 31), (2, 130)], gen) < BOUND[dtype]
    assert w.step([(0, 1), (1, 1), (2, 1)], gen) < BOUND[dtype]            # eager decode first
    bs, dev = 4, torch.device("cuda")
    qsl = torch.arange(bs + 1, dtype=torch.int32, device=dev)               # persistent, as vLLM's
    seq_lens = torch.zeros(bs, dtype=torch.int32, device=dev)
    table = torch.zeros(bs, w.width, dtype=torch.int32, device=dev)
    q_in = [torch.zeros(bs, w.Hq * w.D, dtype=dtype, device=dev) for _ in range(w.layers)]
    k_in = [torch.zeros(bs, w.Hk * w.D, dtype=dtype, device=dev) for _ in range(w.layers)]
    v_in = [torch.zeros(bs, w.Hk * w.D, dtype=dtype, device=dev) for _ in range(w.layers)]
    outs = [torch.zeros(bs, w.Hq * w.D, dtype=dtype, device=dev) for _ in range(w.layers)]

    def prepare():
        """Blocks for the step's token, the persistent tensors, and the builder's metadata; the padding
        row has length 0 (nothing read or written)."""
        for r in live:
            if w.length[r] % PAGE == 0:
                w.table[r, w.length[r] // PAGE] = w.free.pop()
        lens = [w.length[r] + 1 for r in live] + [0]
        seq_lens.copy_(torch.tensor(lens, dtype=torch.int32))
        table.zero_()
        table[:len(live)] = w.table[live, :w.width].to(dev)
        cam = CommonAttentionMetadata(
            query_start_loc=qsl, query_start_loc_cpu=torch.arange(bs + 1, dtype=torch.int32), seq_lens=seq_lens,
            num_reqs=bs, num_actual_tokens=bs, max_query_len=1, max_seq_len=max(lens), block_table_tensor=table,
            slot_mapping=torch.zeros(bs, dtype=torch.int64), seq_lens_cpu_upper_bound=torch.tensor(lens),
            req_idx=np.array([w.slot[r] for r in live] + [0]))
        return w.builder.build(0, cam)

    md = prepare()
    assert md.num_decodes == bs and md.prefill is None
    layer = types.SimpleNamespace(layer_name="l")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(w.layers):
            w.impls[i].forward(layer, q_in[i], k_in[i], v_in[i], w.kv[i], md, output=outs[i])
    torch.cuda.synchronize()
    for step in range(12):
        if step:
            prepare()                                                     # slots into the same buffer
        refs = []
        for i in range(w.layers):
            q, k, v = w.inputs(bs, gen)
            q_in[i].copy_(q)
            k_in[i].copy_(k)
            v_in[i].copy_(v)
            refs.append(w.expected(i, [(r, 1) for r in live], len(live), q, k, v))
        graph.replay()
        torch.cuda.synchronize()
        for r in live:
            w.length[r] += 1
        for i in range(w.layers):
            err = float((outs[i][:len(live)].double().cpu() - refs[i]).norm() / refs[i].norm())
            assert err < BOUND[dtype], (step, i, err)
            assert not outs[i][len(live):].any()                          # the padding row reads nothing
        if step % 4 == 1:
            assert w.step([(r, 1) for r in live], gen) < BOUND[dtype]      # eager steps between replays
        if step % 4 == 3:
            assert w.step([(1, 1), (0, 9)], gen) < BOUND[dtype]
    print(f"graph replays checked; lengths {[w.length[r] for r in live]}", flush=True)
