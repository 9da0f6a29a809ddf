"""The serving integrations' diagnostics and fallback switches (kushkash_amd._serving), forced one by
one on the CPU with the oracle standing in for the kernels, with the reference's meanings
(kushkash/vllm/backend.py:66-67, :80-85, :219-226, :646-658, :738-790; kushkash/sglang/backend.py:45-48):

KUSHKASH_CHECK=<log>   layer 0 of each step checked against torch attention over the cache's own
                       records: one line per call, every request's relative error small, and a wrong
                       output (planted in the oracle) shows up in the log
KUSHKASH_UNPACK=torch  the packed prefill built by torch gives the kernel path's bytes (the oracle's
                       unpack here; the GPU kernel in test_gpu_unpack.py), and serving sessions stay exact
KUSHKASH_SYNC=1        a device synchronization after each attention call, never inside a capture
KUSHKASH_MEM_STATS=N   every N-th packed-prefill step prints the allocator counters
KUSHKASH_PROFILE_STEP=0  vLLM's profiling run reserves no prefill temporaries"""
import types

import numpy as np
import pytest
import torch

import test_sglang
import test_vllm
from _sglang_world import RotatingOracleOps, sglang_standins
from _vllm_world import vllm_standins
from kushkash_amd import _serving
from kushkash_amd._ops import PAGE, pages_touched, record_bytes
from oracle.cpu_ops import OracleOps


@pytest.fixture(scope="module")
def kb():
    with vllm_standins() as backend:
        yield backend


@pytest.fixture(scope="module")
def sg():
    with sglang_standins() as mods:
        yield mods


def _check_lines(path):
    return [l for l in path.read_text().splitlines() if l.startswith("call ")]


@pytest.mark.parametrize("rot", [False, True])
def test_check_log_vllm(kb, monkeypatch, tmp_path, rot):
    monkeypatch.setattr(kb, "Ops", RotatingOracleOps)
    log = tmp_path / "check.log"
    monkeypatch.setenv("KUSHKASH_CHECK", str(log))
    monkeypatch.setattr(_serving, "_check_calls", [0])
    w = test_vllm._engine(kb, monkeypatch, 4, rot)
    worst = test_vllm.serving_session(w, torch.Generator().manual_seed(2), random_steps=6)
    assert worst < 1e-4
    lines = _check_lines(log)
    assert len(lines) >= 8                       # one line per step (layer 0 only)
    assert any(" d" in l for l in lines) and any(" p" in l for l in lines)
    assert max(_serving.max_check_error(l) for l in lines) < 1e-4, lines[:3]


def test_check_log_sglang(sg, monkeypatch, tmp_path):
    monkeypatch.setattr(sg.backend, "Ops", RotatingOracleOps)
    log = tmp_path / "check.log"
    monkeypatch.setenv("KUSHKASH_CHECK", str(log))
    monkeypatch.setattr(_serving, "_check_calls", [0])
    w = test_sglang._server(sg, monkeypatch, 4, rot=True)
    worst = test_sglang.serving_session(w, torch.Generator().manual_seed(3), decode_steps=4, graph_steps=3)
    assert worst < 1e-4
    lines = _check_lines(log)
    assert len(lines) >= 10
    assert max(_serving.max_check_error(l) for l in lines) < 1e-4, lines[:3]


def test_check_log_flags_a_wrong_output(kb, monkeypatch, tmp_path):
    """A decode whose output is off (planted in the oracle standing in for the kernel) shows in the log."""
    class Off(RotatingOracleOps):
        def append_decode(self, *args, **kw):
            super().append_decode(*args, **kw)
            args[3].add_(0.05)                   # out
    monkeypatch.setattr(kb, "Ops", Off)
    log = tmp_path / "check.log"
    monkeypatch.setenv("KUSHKASH_CHECK", str(log))
    monkeypatch.setattr(_serving, "_check_calls", [0])
    w = test_vllm._engine(kb, monkeypatch, 8)
    gen = torch.Generator().manual_seed(4)
    for req, slot in ((0, 1), (1, 3)):
        w.admit(req, slot)
    w.step([(0, 40), (1, 70)], gen)
    w.step([(0, 1), (1, 1)], gen)
    lines = _check_lines(log)
    assert _serving.max_check_error(lines[0]) < 1e-4                 # the prefill step
    assert _serving.max_check_error(lines[1]) > 1e-2                 # the decode step, off by 0.05


def _unpack_case(D, bits, rot, seed):
    """A cache with pages of a few requests, and the packed-plan arrays of one group over them."""
    from kushkash_amd._prefill import pack_plan
    g = torch.Generator().manual_seed(seed)
    H, RB = 2, record_bytes(D, bits)
    ops = RotatingOracleOps("cpu", D, bits, 2)
    history, new = [70, 32, 5, 0], [3, 10, 1, 7]
    blocks = 24
    cache = torch.zeros(blocks, H, RB, dtype=torch.uint8)
    tail = torch.zeros(len(history), H, PAGE, D)
    table = torch.randperm(blocks, generator=g)[:len(history) * 6].view(len(history), 6).to(torch.int32)
    k = torch.randn(sum(history), H, D, generator=g) + 2.0 * torch.linspace(-1, 1, D)
    v = torch.randn(sum(history), H, D, generator=g)
    qsl = torch.tensor([0] + list(np.cumsum(history)), dtype=torch.int32)
    jobs = [(r, p) for r, n in enumerate(history) for p in pages_touched(0, n)]
    slots = torch.arange(len(history), dtype=torch.int32)
    ops.write(k, v, qsl, torch.tensor(history, dtype=torch.int32), slots,
              torch.tensor([j[0] for j in jobs], dtype=torch.int32), torch.tensor([j[1] for j in jobs], dtype=torch.int32),
              cache, table, tail, rot=rot)
    p = pack_plan(new, history, slots.numpy())
    k_new = torch.randn(sum(new), H, D, generator=g)
    v_new = torch.randn(sum(new), H, D, generator=g)
    i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32)
    page_blk = table[i32(p.page_req).long(), i32(p.page_index).long()].contiguous()
    tail_blk = table[i32(p.tail_req).long(), torch.as_tensor([history[r] // PAGE for r in p.tail_req]).long()].contiguous()
    args = (cache, page_blk, i32(p.page_dst), tail_blk, i32(p.tail_info.reshape(-1)), tail, k_new, v_new,
            i32(p.new_dst))
    return ops, args, int(p.key_start[-1]), H


@pytest.mark.parametrize("bits,rot", [(4, False), (4, True), (8, False), (8, True)])
def test_unpack_torch_equals_the_kernel_path(bits, rot):
    D = 64
    ops, args, n_keys, H = _unpack_case(D, bits, rot, seed=bits + rot)
    kp_a, vp_a = torch.full((n_keys, H, D), float("nan")), torch.full((n_keys, H, D), float("nan"))
    kp_b, vp_b = kp_a.clone(), vp_a.clone()
    ops.unpack(*args, kp_a, vp_a, rot)
    _serving.torch_unpack(*args, kp_b, vp_b, D, bits, rot)
    assert torch.equal(kp_a, kp_b) and torch.equal(vp_a, vp_b)


@pytest.mark.parametrize("world", ["vllm", "sglang"])
def test_unpack_torch_serving_sessions(kb, sg, monkeypatch, world):
    monkeypatch.setenv("KUSHKASH_UNPACK", "torch")
    calls = []
    real = _serving.torch_unpack
    monkeypatch.setattr("kushkash_amd._prefill.torch_unpack", lambda *a, **k: (calls.append(1), real(*a, **k)))
    gen = torch.Generator().manual_seed(5)
    if world == "vllm":
        monkeypatch.setattr(kb, "Ops", RotatingOracleOps)
        worst = test_vllm.serving_session(test_vllm._engine(kb, monkeypatch, 4, True), gen, random_steps=6)
    else:
        monkeypatch.setattr(sg.backend, "Ops", RotatingOracleOps)
        worst = test_sglang.serving_session(test_sglang._server(sg, monkeypatch, 8, rot=True), gen,
                                            decode_steps=3, graph_steps=2)
    assert calls, "KUSHKASH_UNPACK=torch never took the torch path"
    assert worst < 1e-4


def test_unpack_mode_names(monkeypatch):
    for value, mode in (("", "kernel"), ("mojo", "kernel"), ("kernel", "kernel"), ("TORCH", "torch")):
        monkeypatch.setenv("KUSHKASH_UNPACK", value) if value else monkeypatch.delenv("KUSHKASH_UNPACK", raising=False)
        assert _serving.unpack_mode() == mode
    monkeypatch.setenv("KUSHKASH_UNPACK", "triton")
    with pytest.raises(ValueError, match="KUSHKASH_UNPACK"):
        _serving.unpack_mode()


def test_sync_switch(monkeypatch):
    calls = []
    monkeypatch.setattr(torch.cuda, "synchronize", lambda device=None: calls.append(device))
    dev = types.SimpleNamespace(is_cuda=True, device="cuda:0")
    for capture in (False, True):
        monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda c=capture: c)
        monkeypatch.delenv("KUSHKASH_SYNC", raising=False)
        _serving.maybe_sync(dev)
        monkeypatch.setenv("KUSHKASH_SYNC", "1")
        _serving.maybe_sync(dev)
    assert calls == ["cuda:0"]                  # switched on, outside a capture: exactly once
    _serving.maybe_sync(types.SimpleNamespace(is_cuda=False, device="cpu"))
    assert len(calls) == 1


def test_mem_stats_switch(monkeypatch, capsys):
    stats = {"num_alloc_retries": 3, "num_ooms": 0, "allocated_bytes.all.current": 5 << 20,
             "reserved_bytes.all.current": 9 << 20, "inactive_split_bytes.all.current": 1 << 20}
    monkeypatch.setattr(torch.cuda, "memory_stats", lambda device=None: stats)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    cuda = types.SimpleNamespace(type="cuda")
    m = _serving.MemStats()
    monkeypatch.delenv("KUSHKASH_MEM_STATS", raising=False)
    assert m.tick(cuda) is None and m.steps == 0              # off by default
    monkeypatch.setenv("KUSHKASH_MEM_STATS", "3")
    printed = [m.tick(cuda) for _ in range(7)]
    assert [p is not None for p in printed] == [False, False, True, False, False, True, False]
    assert "alloc retries 3" in printed[2] and "reserved 9 MiB" in printed[2]
    assert capsys.readouterr().err.count("kushkash mem:") == 2


def test_profile_step_switch(kb, monkeypatch):
    monkeypatch.setattr(kb, "Ops", RotatingOracleOps)
    w = test_vllm._engine(kb, monkeypatch, 4)
    impl = w.impls[0]
    held = []
    monkeypatch.setattr(impl, "_hold_prefill_peak", lambda n, device: held.append(n))
    q = torch.zeros(16, impl.num_heads * impl.head_size)
    kv = torch.zeros(16, impl.num_kv_heads * impl.head_size)
    layer = types.SimpleNamespace(layer_name="model.layers.0.self_attn.attn")
    impl.forward(layer, q, kv, kv, None, None)
    monkeypatch.setenv("KUSHKASH_PROFILE_STEP", "0")
    impl.forward(layer, q, kv, kv, None, None)
    assert held == [16]                          # only the first (default) profiling run reserved
