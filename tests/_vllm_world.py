"""A stand-in for vLLM, for the tests of kushkash_amd.vllm (vLLM is not installed here).

* ``vllm_standins()`` installs modules for the vLLM interfaces the backend uses -- the attention
  backend / impl / metadata-builder base classes, ``CommonAttentionMetadata``, ``AttentionSpec`` and
  ``KVCacheLayout``, ``split_decodes_and_prefills``, the flash-attention availability probe and the
  backend registry -- shaped on the reference's use of them (kushkash/vllm/backend.py:40-53,
  tests/test_vllm_backend_cpu.py:198-206), imports ``kushkash_amd.vllm.backend`` against them and
  removes everything again afterwards.
* ``Engine`` keeps vLLM's state the way model runner V2 fills it: requests in request-state slots
  (req_idx), a block table per request from a shuffled block pool (rows padded, a wider row stride),
  single-token decode rows first, seq_lens that count the step's tokens, the per-layer KV cache as a
  strided [blocks, Hkv, 32, C] slice of a larger allocation. Each step's output is checked against
  float64 attention over the reference quantization of the exact tokens (the references of the
  SGLang tests).
"""
from __future__ import annotations

import contextlib
import enum
import sys
import types
from dataclasses import dataclass
from typing import Generic, TypeVar

import numpy as np
import scipy.linalg
import torch

from _sglang_world import canonical_rotation, causal_gqa, held_in_cache
from kushkash_amd._ops import PAGE, record_bytes

M = TypeVar("M")


class AttentionType:
    DECODER = "decoder"
    ENCODER_DECODER = "encoder_decoder"


class AttentionCGSupport(enum.Enum):
    NEVER = 0
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    ALWAYS = 2


class AttentionBackend:
    pass


class AttentionMetadata:
    pass


class AttentionImpl(Generic[M]):
    pass


class AttentionMetadataBuilder(Generic[M]):
    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        self.kv_cache_spec, self.layer_names, self.vllm_config, self.device = (kv_cache_spec, layer_names,
                                                                              vllm_config, device)
        self.reorder_batch_threshold = None

    def _init_reorder_batch_threshold(self, threshold, supports_spec_as_decode=False):
        self.reorder_batch_threshold = threshold


@dataclass
class CommonAttentionMetadata:
    query_start_loc: torch.Tensor
    query_start_loc_cpu: torch.Tensor
    seq_lens: torch.Tensor
    num_reqs: int
    num_actual_tokens: int
    max_query_len: int
    max_seq_len: int
    block_table_tensor: torch.Tensor
    slot_mapping: torch.Tensor
    seq_lens_cpu_upper_bound: torch.Tensor | None = None
    req_idx: np.ndarray | None = None


@dataclass
class AttentionSpec:
    block_size: int
    num_kv_heads: int
    head_size: int
    dtype: torch.dtype
    state_content_bytes: int | None = None


class KVCacheLayout(enum.Enum):
    NHD = "NHD"
    LBHNC = "LBHNC"


def split_decodes_and_prefills(cam, decode_threshold=1):
    """(decode requests, prefill requests, decode tokens, prefill tokens): the leading requests with
    at most decode_threshold query tokens are decodes (the batch is ordered that way)."""
    qsl = cam.query_start_loc_cpu[:cam.num_reqs + 1]
    qlen = (qsl[1:] - qsl[:-1]).tolist()
    nd = 0
    while nd < len(qlen) and qlen[nd] <= decode_threshold:
        nd += 1
    dec_tokens = int(qsl[nd])
    return nd, cam.num_reqs - nd, dec_tokens, int(qsl[-1]) - dec_tokens


_CONFIG = {"current": None}


def get_current_vllm_config():
    return _CONFIG["current"]


def _modules() -> dict:
    names = ("vllm", "vllm.config", "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backend",
             "vllm.v1.attention.backends", "vllm.v1.attention.backends.fa_utils", "vllm.v1.attention.backends.utils",
             "vllm.v1.kv_cache_interface")
    mods = {n: types.ModuleType(n) for n in names}
    mods["vllm.config"].get_current_vllm_config = get_current_vllm_config
    b = mods["vllm.v1.attention.backend"]
    for cls in (AttentionBackend, AttentionCGSupport, AttentionImpl, AttentionMetadata, AttentionMetadataBuilder,
                AttentionType, CommonAttentionMetadata):
        setattr(b, cls.__name__, cls)
    mods["vllm.v1.attention.backends.fa_utils"].is_flash_attn_varlen_func_available = lambda: False
    mods["vllm.v1.attention.backends.utils"].split_decodes_and_prefills = split_decodes_and_prefills
    mods["vllm.v1.kv_cache_interface"].AttentionSpec = AttentionSpec
    mods["vllm.v1.kv_cache_interface"].KVCacheLayout = KVCacheLayout
    return mods


def _drop_backend_modules():
    import kushkash_amd.vllm as kv
    for name in [n for n in sys.modules if n.startswith("kushkash_amd.vllm.")]:
        sys.modules.pop(name)
        short = name.rsplit(".", 1)[1]
        if hasattr(kv, short):
            delattr(kv, short)


@contextlib.contextmanager
def vllm_standins():
    """Yields the backend module imported against the stand-ins; sys.modules is restored afterwards."""
    mods = _modules()
    saved = {name: sys.modules.get(name) for name in mods}
    sys.modules.update(mods)
    try:
        _drop_backend_modules()
        from kushkash_amd.vllm import backend
        yield backend
    finally:
        _drop_backend_modules()
        for name, old in saved.items():
            if old is None:
                sys.modules.pop(name, None)
            else:
                sys.modules[name] = old


def vllm_config(max_seqs: int, max_len: int, dtype: torch.dtype, max_tokens: int = 512):
    return types.SimpleNamespace(
        model_config=types.SimpleNamespace(dtype=dtype, max_model_len=max_len),
        scheduler_config=types.SimpleNamespace(max_num_seqs=max_seqs, max_num_batched_tokens=max_tokens),
        speculative_config=None, parallel_config=types.SimpleNamespace(use_ubatching=False))


class Engine:
    """vLLM-like state around one KushAttentionImpl and its metadata builder."""

    def __init__(self, kb, *, device, dtype, bits, Hq=6, Hk=2, D=64, layers=2, max_seqs=8, width=24, blocks=160,
                 seed=1):
        self.kb, self.device, self.dtype, self.bits = kb, torch.device(device), dtype, bits
        self.Hq, self.Hk, self.D, self.layers, self.width = Hq, Hk, D, layers, width
        self.cfg = vllm_config(max_seqs, width * PAGE, dtype)
        _CONFIG["current"] = self.cfg
        # one impl per attention layer, as vLLM builds them: each holds its layer's K tails
        self.impls = [kb.KushAttentionImpl(Hq, D, D ** -0.5, num_kv_heads=Hk) for _ in range(layers)]
        self.impl = self.impls[0]
        spec = AttentionSpec(block_size=PAGE, num_kv_heads=Hk, head_size=D, dtype=dtype)
        self.builder = kb.KushMetadataBuilder(spec, ["l0"], self.cfg, self.device)
        C = record_bytes(D, bits) // PAGE
        # per layer: a strided [blocks, Hkv, 32, C] slice of a wider allocation, as vLLM may hand it over
        self.kv = [torch.zeros(blocks, Hk * PAGE * C + 256, dtype=torch.uint8, device=self.device)[:, :Hk * PAGE * C]
                   .view(blocks, Hk, PAGE, C) for _ in range(layers)]
        g = torch.Generator().manual_seed(seed)
        self.free = torch.randperm(blocks, generator=g).tolist()
        self.table = torch.zeros(max_seqs * 2, width, dtype=torch.int32)
        self.length: dict[int, int] = {}
        self.slot: dict[int, int] = {}
        self.tokens: dict[tuple[int, int], tuple[torch.Tensor, torch.Tensor]] = {}
        self.h = (torch.from_numpy(scipy.linalg.hadamard(D)).double() / D ** 0.5) if self.impl.rot else None
        self.rotate = canonical_rotation(D, dtype) if self.impl.rot else None

    def admit(self, req: int, slot: int) -> None:
        """A new request in request-state slot `slot` (vLLM's req_idx)."""
        self.slot[req], self.length[req] = slot, 0

    def finish(self, req: int) -> None:
        """The request leaves; its blocks return to the pool and its slot may be reused."""
        pages = -(-self.length[req] // PAGE)
        self.free += self.table[req, :pages].tolist()
        for layer in range(self.layers):
            self.tokens.pop((layer, req), None)
        del self.length[req], self.slot[req]

    def metadata(self, plan):
        """CommonAttentionMetadata of a step: plan = [(request, new tokens)], decodes first."""
        reqs = [r for r, _ in plan]
        ql = [c for _, c in plan]
        for r, c in plan:                                        # blocks for the new tokens
            have, need = -(-self.length[r] // PAGE), -(-(self.length[r] + c) // PAGE)
            for p in range(have, need):
                self.table[r, p] = self.free.pop()
        qsl = torch.tensor(np.concatenate([[0], np.cumsum(ql)]), dtype=torch.int32)
        sl = torch.tensor([self.length[r] + c for r, c in plan], dtype=torch.int32)
        n, N = len(plan), int(qsl[-1])
        bt = torch.zeros(n + 2, self.width + 3, dtype=torch.int32, device=self.device)[:, :self.width]
        bt[:n] = self.table[reqs].to(self.device)                # padded rows, a wider row stride
        return CommonAttentionMetadata(
            query_start_loc=qsl.to(self.device), query_start_loc_cpu=qsl, seq_lens=sl.to(self.device), num_reqs=n,
            num_actual_tokens=N, max_query_len=max(ql), max_seq_len=int(sl.max()), block_table_tensor=bt[:n],
            slot_mapping=torch.zeros(N, dtype=torch.int64), seq_lens_cpu_upper_bound=sl,
            req_idx=np.array([self.slot[r] for r in reqs]))

    def inputs(self, rows: int, gen: torch.Generator):
        q = torch.randn(rows, self.Hq * self.D, generator=gen)
        k = torch.randn(rows, self.Hk * self.D, generator=gen) + 3.0 * torch.linspace(-1, 1, self.D).repeat(self.Hk)
        v = torch.randn(rows, self.Hk * self.D, generator=gen)
        return [x.to(self.dtype) for x in (q, k, v)]

    def expected(self, layer, plan, nd, q, k, v) -> torch.Tensor:
        """Reference [T, Hq * D] (float64) of the step; records the new tokens in the shadow."""
        outs, a = [], 0
        empty = torch.zeros(0, self.Hk, self.D, dtype=torch.float64)
        for i, (r, c) in enumerate(plan):
            K0, V0 = self.tokens.get((layer, r), (empty, empty))
            kn = k[a:a + c].double().view(c, self.Hk, self.D)
            vn = v[a:a + c].double().view(c, self.Hk, self.D)
            Kall, Vall = torch.cat([K0, kn]), torch.cat([V0, vn])
            self.tokens[(layer, r)] = (Kall, Vall)
            if i < nd:                                           # decode: the cache including the new token
                Kq, Vq = held_in_cache(Kall, Vall, self.bits, self.rotate, self.h)
            else:                                                # prefill: cached history, then the chunk exact
                Kh, Vh = held_in_cache(K0, V0, self.bits, self.rotate, self.h)
                Kq, Vq = torch.cat([Kh, kn]), torch.cat([Vh, vn])
            outs.append(causal_gqa(q[a:a + c].double().view(c, self.Hq, self.D), Kq, Vq, K0.shape[0], self.D ** -0.5))
            a += c
        return torch.cat(outs).reshape(-1, self.Hq * self.D)

    def step(self, plan, gen: torch.Generator, pad: int = 3) -> float:
        """One step over every layer; returns the worst relative error (Frobenius) of any layer."""
        cam = self.metadata(plan)
        md = self.last_md = self.builder.build(0, cam)
        N = cam.num_actual_tokens
        worst = 0.0
        for layer in range(self.layers):
            q, k, v = self.inputs(N + pad, gen)                  # vLLM pads the token rows
            out = torch.zeros(N + pad, self.Hq * self.D, dtype=self.dtype, device=self.device)
            self.impls[layer].forward(types.SimpleNamespace(layer_name=f"model.layers.{layer}.self_attn.attn"),
                              q.to(self.device), k.to(self.device), v.to(self.device), self.kv[layer], md, output=out)
            ref = self.expected(layer, plan, md.num_decodes, q, k, v)
            worst = max(worst, float((out[:N].double().cpu() - ref).norm() / ref.norm()))
            assert not out[N:].any(), "padded rows were written"
        for r, c in plan:
            self.length[r] += c
        return worst
