"""Generation loop for Hugging Face causal LMs on a KushHFCache, with the decode step replayed from a
HIP graph. Contract: kushkash/_generate.py:1-173 (same signature, stats and stopping rules).

    tokens = kushkash_amd.generate(model, input_ids, max_new_tokens=256, bits=4)

Against model.generate: the prompt is prefilled in chunks of `prefill_chunk` tokens (later chunks
attend over the quantized history), and after WARMUP_STEPS eager steps the whole decode step (all
layers: projections, MLPs, the append and decode kernels) is captured once as a HIP graph and
replayed. Greedy or temperature / top-k sampling, optional EOS, equal-length batches.
"""
from __future__ import annotations

import time

import torch

from .hf import NAME, KushHFCache, enable

WARMUP_STEPS = 2      # eager decode steps (on a side stream) before the capture
EOS_LAG = 2           # with EOS: the host runs at most this many steps ahead of the `done` readback


def _pick(logits: torch.Tensor, do_sample: bool, temperature: float, top_k: int) -> torch.Tensor:
    if not do_sample:
        return logits.argmax(-1)
    logits = logits.float() / max(temperature, 1e-5)
    if top_k:
        logits = logits.masked_fill(logits < logits.topk(top_k, -1).values[:, -1:], float("-inf"))
    return torch.multinomial(torch.softmax(logits, -1), 1)[:, 0]


class _EosWatch:
    """EOS stop without a host sync per token (_generate.py:87-115): `done` is copied to pinned host
    memory asynchronously and read once the copy has landed, or waited for once it is EOS_LAG steps
    old (graph replays are queued far faster than the GPU runs them, so an unbounded host would
    queue every step before the GPU reached the EOS). Rows already done keep emitting EOS."""

    def __init__(self, eos: torch.Tensor, batch: int, device: torch.device):
        self.eos = eos
        self.done = torch.zeros(batch, dtype=torch.bool, device=device)
        self.host = torch.zeros(batch, dtype=torch.bool, pin_memory=True)
        self.ev = torch.cuda.Event()
        self.pending, self.at = False, 0

    def stop(self, tok: torch.Tensor, step: int) -> bool:
        self.done |= torch.isin(tok, self.eos)
        if self.pending and (self.ev.query() or step - self.at >= EOS_LAG):
            self.ev.synchronize()
            self.pending = False
            if bool(self.host.all()):
                return True
        if not self.pending:
            self.host.copy_(self.done, non_blocking=True)
            self.ev.record()
            self.pending, self.at = True, step
        return False


@torch.no_grad()
def generate(model, input_ids: torch.Tensor, max_new_tokens: int, *, bits: int = 4,
             cache: KushHFCache | None = None, prefill_chunk: int = 1024, cuda_graph: bool | str = "auto",
             eos_token_id: int | list[int] | None = None, do_sample: bool = False,
             temperature: float = 1.0, top_k: int = 0, stats: dict | None = None) -> torch.Tensor:
    """Returns [B, prompt + generated] token ids; rows that hit EOS are padded with EOS.

    Args:
        cache: optional fresh KushHFCache (to read `cache.memory()` afterwards).
        prefill_chunk: prompt tokens per forward during the prefill.
        cuda_graph: capture and replay the decode step as a HIP graph. "auto": keep the graph only if
            its replay is > 10 % faster than an eager step (median of 3 timed replays), and step
            eagerly if the capture runs out of memory; True: always keep it; False: never capture.
        stats: optional dict, filled with prefill_s, prefill_history_attn_s, decode_s, decode_tokens,
            graph, eager_step_ms, graph_step_ms.
    """
    if model.config._attn_implementation != NAME:
        enable(model)
    dev = input_ids.device
    if dev.type != "cuda":
        raise ValueError("kushkash_amd.generate runs on the GPU (input_ids on a 'cuda' device under ROCm)")
    B, T0 = input_ids.shape
    total = T0 + max_new_tokens
    cache = cache if cache is not None else KushHFCache(model.config, bits=bits, max_length=total)
    eos = torch.tensor([eos_token_id] if isinstance(eos_token_id, int) else list(eos_token_id or []),
                       dtype=torch.long, device=dev)
    watch = _EosWatch(eos, B, dev) if eos.numel() else None

    def forward(ids, pos):
        return model(input_ids=ids, position_ids=pos, past_key_values=cache, use_cache=True,
                     logits_to_keep=1).logits[:, -1]

    def sync():
        torch.cuda.synchronize(dev)

    t0 = time.perf_counter()
    for c0 in range(0, T0, prefill_chunk):
        if stats is not None and cache.kv is not None and cache.kv.profile is None:
            cache.kv.profile = []              # time the chunks that attend over history
        ids = input_ids[:, c0:c0 + prefill_chunk]
        logits = forward(ids, torch.arange(c0, c0 + ids.shape[1], device=dev).expand(B, -1))
    tok = _pick(logits, do_sample, temperature, top_k)
    sync()
    t1 = time.perf_counter()

    kv = cache.kv
    kv.freeze(total)                           # every page mapped, split-K fixed: steps allocate nothing
    ids_in = torch.zeros(B, 1, dtype=input_ids.dtype, device=dev)
    pos_in = torch.zeros(B, 1, dtype=torch.long, device=dev)
    want_graph = bool(cuda_graph)
    graph, logits_out = None, None
    side = torch.cuda.Stream(dev) if want_graph else None
    eager_ms, graph_ms = None, []
    out, n = [tok], T0
    for i in range(1, max_new_tokens):
        if watch is not None and watch.stop(tok, i):
            break
        ids_in.copy_(tok.view(B, 1))
        pos_in.fill_(n)
        if graph is not None:
            timed = cuda_graph == "auto" and len(graph_ms) < 3
            if timed:
                sync()
                ts = time.perf_counter()
            graph.replay()
            kv.advance(1)
            logits = logits_out
            if timed:
                sync()
                graph_ms.append((time.perf_counter() - ts) * 1e3)
                if len(graph_ms) == 3 and sorted(graph_ms)[1] > 0.9 * eager_ms:
                    graph, logits_out, want_graph = None, None, False      # not worth its memory
        elif want_graph and i > WARMUP_STEPS:
            lens = list(kv._len)                # the capture records the step, it does not run it
            try:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    logits_out = forward(ids_in, pos_in)
            except torch.OutOfMemoryError:
                graph, logits_out, want_graph = None, None, False
            finally:
                kv._len = lens
            if graph is None:
                torch.cuda.empty_cache()
                logits = forward(ids_in, pos_in)
            else:
                graph.replay()
                kv.advance(1)
                logits = logits_out
        elif want_graph:                        # warm-up steps on a side stream, as torch's capture asks
            sync()
            ts = time.perf_counter()
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                logits = forward(ids_in, pos_in)
            torch.cuda.current_stream(dev).wait_stream(side)
            sync()
            eager_ms = (time.perf_counter() - ts) * 1e3
        else:
            logits = forward(ids_in, pos_in)
        n += 1
        tok = _pick(logits, do_sample, temperature, top_k)
        if watch is not None:
            tok = torch.where(watch.done, eos[0], tok)
        out.append(tok)
    sync()
    if stats is not None:
        hist = sum(a.elapsed_time(b) for a, b in kv.profile) / 1e3 if kv.profile else 0.0
        kv.profile = None
        stats.update(prefill_s=t1 - t0, prefill_history_attn_s=hist, decode_s=time.perf_counter() - t1,
                     decode_tokens=B * (len(out) - 1), graph=graph is not None, eager_step_ms=eager_ms,
                     graph_step_ms=sorted(graph_ms)[len(graph_ms) // 2] if graph_ms else None)
    del graph, logits_out
    return torch.cat([input_ids, torch.stack(out, 1)], 1)
