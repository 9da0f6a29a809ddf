"""A stand-in for SGLang, for the tests of kushkash_amd.sglang (SGLang is not installed here).

* ``sglang_standins()`` installs modules for the two SGLang classes the backend subclasses
  (``AttentionBackend``, ``MHATokenToKVPool``), imports ``kushkash_amd.sglang.pool`` / ``.backend``
  against them and removes everything again afterwards (the way the reference tests its backend
  without SGLang: tests/test_sglang_backend_cpu.py:19-62).
* ``Server`` keeps SGLang's state the way SGLang fills it: a page allocator over token slots,
  ``req_to_token``, request-pool slots, seq_lens that already count the step's tokens, radix-cache
  prefixes shared between requests, padded decode batches. Every step's output is checked against
  attention over an independent shadow of the exact tokens, quantized the way the cache must hold
  them (restated from the reference test's ``ref_dequant``, with scipy's Hadamard matrix for the
  rotation), in float64.
* ``RotatingOracleOps`` is the CPU oracle with the GPU ``Ops``' in-kernel rotation argument, for the
  CPU tests.
"""
from __future__ import annotations

import contextlib
import sys
import types

import numpy as np
import scipy.linalg
import torch

from _harness import ref_dequant
from kushkash_amd._ops import PAGE
from oracle.cpu_ops import OracleOps
from oracle.cpu_ops import call as oracle_call

_STANDIN_NAMES = ("sglang", "sglang.srt", "sglang.srt.layers", "sglang.srt.layers.attention",
                  "sglang.srt.layers.attention.base_attn_backend", "sglang.srt.mem_cache",
                  "sglang.srt.mem_cache.memory_pool")


class AttentionBackend:
    """SGLang's backend base class, as far as the backend uses it."""

    def __init__(self):
        pass


class MHATokenToKVPool:
    """SGLang's MHA pool base class: stores the geometry, then lets the subclass create its buffers."""

    def __init__(self, size, page_size, head_num, head_dim, layer_num, device, start_layer=0):
        self.size, self.page_size, self.head_num, self.head_dim = size, page_size, head_num, head_dim
        self.v_head_dim, self.layer_num, self.device, self.start_layer = head_dim, layer_num, device, start_layer
        self.memory_saver_adapter = None
        self._create_buffers()

    def _init_data_ptrs_and_strides(self):
        self.data_ptrs = [t.data_ptr() for t in self.k_buffer]


def _drop_backend_modules():
    import kushkash_amd.sglang as ks
    for name in [n for n in sys.modules if n.startswith("kushkash_amd.sglang.")]:
        sys.modules.pop(name)
        short = name.rsplit(".", 1)[1]
        if hasattr(ks, short):
            delattr(ks, short)


@contextlib.contextmanager
def sglang_standins():
    """Yields a namespace with the backend and pool modules imported against the stand-ins."""
    mods = {name: types.ModuleType(name) for name in _STANDIN_NAMES}
    mods["sglang.srt.layers.attention.base_attn_backend"].AttentionBackend = AttentionBackend
    mods["sglang.srt.mem_cache.memory_pool"].MHATokenToKVPool = MHATokenToKVPool
    with _patched_modules(mods):
        _drop_backend_modules()
        try:
            from kushkash_amd.sglang import backend, pool
            yield types.SimpleNamespace(backend=backend, pool=pool)
        finally:
            _drop_backend_modules()


@contextlib.contextmanager
def _patched_modules(mods: dict):
    saved = {name: sys.modules.get(name) for name in mods}
    sys.modules.update(mods)
    try:
        yield
    finally:
        for name, old in saved.items():
            if old is None:
                sys.modules.pop(name, None)
            else:
                sys.modules[name] = old


class RotatingOracleOps(OracleOps):
    """OracleOps (fp32, CPU) with the rot argument of the GPU Ops: the rows a write or append stores
    are rotated first (the oracle's Walsh-Hadamard transform), the decode rotates q and its output
    back; unpack takes rot already. Test infrastructure."""

    def _rotated(self, x: torch.Tensor) -> torch.Tensor:
        y = x.contiguous().clone()
        return self.fwht(y, y)

    def append(self, k, v, seq_lens, tail_idx, cache, block_table, tail_k, pos_offset, advance, *, rot=False):
        if rot:
            k, v = self._rotated(k), self._rotated(v)
        super().append(k, v, seq_lens, tail_idx, cache, block_table, tail_k, pos_offset, advance)

    def write(self, k, v, query_start_loc, seq_lens, tail_idx, job_seq, job_page, cache, block_table, tail_k, *,
              fused=False, rot=False):
        if rot:
            k, v = self._rotated(k), self._rotated(v)
        super().write(k, v, query_start_loc, seq_lens, tail_idx, job_seq, job_page, cache, block_table, tail_k,
                      fused=fused)

    def decode(self, q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits=1, work=None, *,
               waves=None, order=None, rot=False):
        if rot:
            q = self._rotated(q)
        super().decode(q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits, work)
        if rot:
            self.fwht(out, out)

    def append_decode(self, k, v, q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits=1,
                      work=None, *, waves=None, order=None, rot=False):
        self.append(k, v, seq_lens, tail_idx, cache, block_table, tail_k, -1, False, rot=rot)
        self.decode(q, out, cache, block_table, seq_lens, tail_idx, tail_k, scale, n_splits, work, rot=rot)


class Mode:
    """SGLang's ForwardMode, as far as the backend asks."""

    def __init__(self, decode: bool, idle: bool = False, verify: bool = False):
        self.decode, self.idle, self.verify = decode, idle, verify

    def is_idle(self):
        return self.idle

    def is_decode(self):
        return self.decode

    def is_target_verify(self):
        return self.verify

    def is_draft_extend_v2(self):
        return False

    def __repr__(self):
        return "DECODE" if self.decode else "EXTEND"


class Layer:
    """A RadixAttention layer's attributes."""

    def __init__(self, layer_id, Hq, Hk, D):
        self.layer_id, self.tp_q_head_num, self.tp_k_head_num, self.qk_head_dim = layer_id, Hq, Hk, D
        self.scaling = D ** -0.5
        self.logit_cap, self.sliding_window_size, self.is_cross_attention = 0.0, -1, False


def canonical_rotation(D: int, dtype: torch.dtype):
    """Rows [..., D] -> the same rows rotated as the kernels rotate before they quantize: the canonical
    Walsh-Hadamard transform in fp32 (the oracle's, which is checked against the dense Hadamard product),
    rounded to the model dtype; returned as float64."""
    def rotate(x: torch.Tensor) -> torch.Tensor:
        y = x.float().contiguous().clone()
        if y.numel():
            oracle_call("kush_cpu_fwht", D, y.data_ptr(), y.numel() // D)
        return y.to(dtype).double()
    return rotate


def held_in_cache(K: torch.Tensor, V: torch.Tensor, bits: int, rotate=None, h: torch.Tensor | None = None):
    """The K, V [n, Hk, D] a cache hands back for exact tokens K, V (values of the model dtype), in model
    space: the K rows of every completed page quantized per channel across the page's 32 tokens, the
    rows of the unfinished page as they are, every V row quantized per token. With a rotation the
    cache holds rotate(K), rotate(V), handed back through the orthonormal Hadamard matrix h. The
    rotation is the format's own and the quantizer works in fp32 like the kernels, so every code
    matches theirs: a rotation or a quantizer that rounds differently moves a value across a rounding
    boundary now and then, which changes its code by one level."""
    if rotate is not None:
        K, V = rotate(K), rotate(V)
    done = K.shape[0] - K.shape[0] % PAGE
    pages = K[:done].float().unflatten(0, (-1, PAGE))                    # [pages, 32, Hk, D]
    k_held = torch.cat([ref_dequant(pages, bits, 1).flatten(0, 1).double(), K[done:]])
    v_held = ref_dequant(V.float(), bits, -1).double()
    if rotate is not None:
        k_held, v_held = k_held @ h, v_held @ h
    return k_held, v_held


def causal_gqa(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, first: int, scale: float) -> torch.Tensor:
    """Attention of T queries q [T, Hq, D] over keys K, V [n, Hk, D], float64 on the CPU: q head i reads
    kv head i // (Hq / Hk); query t is at position first + t and sees the keys up to it."""
    T, Hq, D = q.shape
    Hk = K.shape[1]
    qg = q.reshape(T, Hk, Hq // Hk, D)
    logits = torch.einsum("tkgd,nkd->kgtn", qg, K) * scale
    hidden = torch.arange(K.shape[0])[None, :] > (first + torch.arange(T))[:, None]      # [T, n]
    weights = logits.masked_fill(hidden, float("-inf")).softmax(dim=-1)
    return torch.einsum("kgtn,nkd->tkgd", weights, V).reshape(T, Hq, D)


class Server:
    """SGLang-like state around one KushSGLangBackend."""

    def __init__(self, sg, *, device, dtype, bits, Hq=4, Hk=2, D=64, layers=2, slots=8, context=512, pages=64,
                 seed=1):
        self.sg, self.device, self.dtype, self.bits = sg, torch.device(device), dtype, bits
        self.Hq, self.Hk, self.D, self.layers = Hq, Hk, D, layers
        self.pool = sg.pool.KushPool(size=(pages - 1) * PAGE, page_size=PAGE, head_num=Hk, head_dim=D,
                                     layer_num=layers, device=self.device)
        self.req_to_token = torch.zeros(slots, context, dtype=torch.int32, device=self.device)
        runner = types.SimpleNamespace(token_to_kv_pool=self.pool,
                                       req_to_token_pool=types.SimpleNamespace(req_to_token=self.req_to_token),
                                       model_config=types.SimpleNamespace(dtype=dtype))
        self.backend = sg.backend.KushSGLangBackend(runner)
        self.backend.G = Hq // Hk                      # the stand-ins have no parallel config to read it from
        self.h = (torch.from_numpy(scipy.linalg.hadamard(D)).double() / D ** 0.5) if self.backend.rot else None
        self.rotate = canonical_rotation(D, dtype) if self.backend.rot else None
        g = torch.Generator().manual_seed(seed)
        self.free = (torch.randperm(pages - 1, generator=g) + 1).tolist()      # page 0: SGLang's padding page
        self.length: dict[int, int] = {}
        self.tokens: dict[tuple[int, int], tuple[torch.Tensor, torch.Tensor]] = {}   # (layer, slot) -> exact K, V

    # ---------------------------------------------------------------- SGLang's bookkeeping
    def grow(self, slot: int, n: int) -> None:
        """Token slots for n more tokens of request `slot`: whole pages from the free list, as many as
        the new length needs beyond the pages the request holds."""
        have = self.length.get(slot, 0)
        held, needed = -(-have // PAGE), -(-(have + n) // PAGE)
        for p in range(held, needed):
            first = self.free.pop() * PAGE
            self.req_to_token[slot, p * PAGE:(p + 1) * PAGE] = torch.arange(first, first + PAGE, dtype=torch.int32)
        self.length[slot] = have + n

    def share(self, src: int, dst: int, n: int) -> None:
        """A radix-cache hit: request dst starts with the first n (whole pages) tokens of src."""
        assert n % PAGE == 0
        self.req_to_token[dst, :n] = self.req_to_token[src, :n]
        self.length[dst] = n
        for layer in range(self.layers):
            K, V = self.tokens[(layer, src)]
            self.tokens[(layer, dst)] = (K[:n].clone(), V[:n].clone())

    def batch(self, slots, counts, decode: bool, pad: int = 0):
        """A ForwardBatch; `pad` padded rows (request slot 0, seq_len 1) as a graph replay has them."""
        lens = [self.length[s] for s in slots]
        req = torch.tensor(list(slots) + [0] * pad, dtype=torch.int64)
        sl = torch.tensor(lens + [1] * pad, dtype=torch.int64)
        return types.SimpleNamespace(forward_mode=Mode(decode), req_pool_indices=req.to(self.device),
                                     req_pool_indices_cpu=req, seq_lens=sl.to(self.device), seq_lens_cpu=sl,
                                     extend_seq_lens_cpu=list(counts),
                                     extend_prefix_lens_cpu=[n - c for n, c in zip(lens, counts)])

    # ---------------------------------------------------------------- one step
    def inputs(self, rows: int, gen: torch.Generator):
        """q, k, v of one layer for `rows` tokens, in the model dtype (k with per-channel offsets, so
        the K pages quantize per channel for real)."""
        q = torch.randn(rows, self.Hq * self.D, generator=gen)
        k = torch.randn(rows, self.Hk * self.D, generator=gen) + 3.0 * torch.linspace(-1, 1, self.D).repeat(self.Hk)
        v = torch.randn(rows, self.Hk * self.D, generator=gen)
        return [x.to(self.dtype) for x in (q, k, v)]

    def expected(self, layer: int, slots, counts, q, k, v, decode: bool, before) -> torch.Tensor:
        """Reference output [T, Hq * D] (float64) of a step whose inputs were q, k, v; records the new
        tokens in the shadow. before: each request's length before the step."""
        outs, a = [], 0
        empty = torch.zeros(0, self.Hk, self.D, dtype=torch.float64)
        for s, c, n0 in zip(slots, counts, before):
            K0, V0 = self.tokens.get((layer, s), (empty, empty))
            kn = k[a:a + c].double().view(c, self.Hk, self.D)
            vn = v[a:a + c].double().view(c, self.Hk, self.D)
            Kall, Vall = torch.cat([K0, kn]), torch.cat([V0, vn])
            self.tokens[(layer, s)] = (Kall, Vall)
            qs = q[a:a + c].double().view(c, self.Hq, self.D)
            if decode:                                 # the whole cache, the new token included
                Kq, Vq = held_in_cache(Kall, Vall, self.bits, self.rotate, self.h)
            else:                                      # the cached history, then the chunk exact
                Kh, Vh = held_in_cache(K0, V0, self.bits, self.rotate, self.h)
                Kq, Vq = torch.cat([Kh, kn]), torch.cat([Vh, vn])
            outs.append(causal_gqa(qs, Kq, Vq, n0, self.D ** -0.5))
            a += c
        return torch.cat(outs).reshape(-1, self.Hq * self.D)

    def step(self, slots, counts, decode: bool, gen: torch.Generator, pad: int | None = None) -> float:
        """One step over every layer through the backend (eager metadata, or the graph-metadata path with
        `pad` padded rows); returns the worst relative error (Frobenius) against the reference."""
        before = [self.length.get(s, 0) for s in slots]
        for s, c in zip(slots, counts):
            self.grow(s, c)
        fb = self.batch(slots, counts, decode, pad or 0)
        if pad is None:
            self.backend.init_forward_metadata(fb)
        else:
            self.backend.init_forward_metadata_out_graph(fb)
        T = sum(counts)
        worst = 0.0
        for layer in range(self.layers):
            q, k, v = self.inputs(T + (pad or 0), gen)
            run = self.backend.forward_decode if decode else self.backend.forward_extend
            out = run(q.to(self.device), k.to(self.device), v.to(self.device), Layer(layer, self.Hq, self.Hk, self.D),
                      fb)[:T]
            ref = self.expected(layer, slots, counts, q, k, v, decode, before)
            worst = max(worst, float((out.double().cpu() - ref).norm() / ref.norm()))
        return worst


def pack_plan_is_exact(plan, new_tokens, history, slots) -> None:
    """Assert that a packed-prefill plan places every key of every request exactly once, in order:
    request r's history pages, then its partial page's tokens, then its new tokens."""
    q = np.asarray(new_tokens)
    h = np.asarray(history)
    starts = np.concatenate([[0], np.cumsum(q + h)])
    assert (plan.key_start == starts).all()
    source = {}                                        # packed row -> what fills it
    for i in range(len(plan.page_req)):
        r, p, d = int(plan.page_req[i]), int(plan.page_index[i]), int(plan.page_dst[i])
        for t in range(PAGE):
            source.setdefault(d + t, []).append(("page", r, p * PAGE + t))
    for i, r in enumerate(plan.tail_req):
        first, n, slot = (int(x) for x in plan.tail_info[i])
        assert slot == slots[r] and n == h[r] % PAGE
        for t in range(n):
            source.setdefault(first + t, []).append(("tail", int(r), h[r] // PAGE * PAGE + t))
    token = 0
    for r in range(len(q)):
        for t in range(q[r]):
            source.setdefault(int(plan.new_dst[token]), []).append(("new", r, h[r] + t))
            token += 1
    assert sorted(source) == list(range(int(starts[-1])))
    for row, found in source.items():
        assert len(found) == 1, (row, found)
        kind, r, pos = found[0]
        assert row == starts[r] + pos, (row, found)           # position pos of request r, in order
        assert kind == ("new" if pos >= h[r] else "page" if pos < h[r] // PAGE * PAGE else "tail"), (row, found)
