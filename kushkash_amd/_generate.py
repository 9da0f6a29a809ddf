"""Generation loop for Hugging Face causal LMs on a KushHFCache, the decode step replayed from a HIP
graph. Signature, stats and stopping rule: the reference's generate (kushkash/_generate.py:33-173).

    tokens = kushkash_amd.generate(model, input_ids, max_new_tokens=256, bits=4)

Prefill runs in chunks of prefill_chunk tokens (later chunks attend over the quantized history).
Decode runs one token per step through _DecodeStep, which owns the step's static inputs and, after
WARMUP_STEPS eager steps, captures the whole step (all layers: projections, MLPs, the fused append +
decode launches) once and replays it. EOS stopping never synchronizes per token: _StopSignal copies
each step's "all rows done" flags to pinned host memory and reads them EOS_LAG steps later. Greedy or
temperature / top-k sampling; equal-length batches.
"""
from __future__ import annotations

import time

import torch

from .hf import NAME, KushHFCache, enable

WARMUP_STEPS = 2      # eager steps (on a side stream, as torch's capture asks) before the capture
EOS_LAG = 2           # the host reads a step's EOS flags this many steps after queuing it


def _pick(logits: torch.Tensor, do_sample: bool, temperature: float, top_k: int) -> torch.Tensor:
    """Next token per row: argmax, or a sample from softmax(logits / temperature) restricted to the
    top_k largest logits when top_k > 0 (_generate.py:23-30)."""
    if not do_sample:
        return logits.argmax(-1)
    z = logits.float() / max(temperature, 1e-5)
    if top_k:
        top = z.topk(min(top_k, z.shape[-1]), dim=-1)
        choice = torch.multinomial(torch.softmax(top.values, -1), 1)
        return top.indices.gather(-1, choice)[:, 0]
    return torch.multinomial(torch.softmax(z, -1), 1)[:, 0]


class _StopSignal:
    """All-rows-done detection without a host synchronization per token. Each step's `done` flags go
    to a pinned host slot of a ring by an asynchronous copy, with an event; the host reads the slot of
    the step EOS_LAG steps back (waiting for its copy if the GPU is behind), so it queues at most
    EOS_LAG steps past the step that finished every row and the GPU never idles for the check. Rows
    already done keep emitting EOS."""

    def __init__(self, eos: torch.Tensor, batch: int, device: torch.device):
        self.eos = eos
        self.done = torch.zeros(batch, dtype=torch.bool, device=device)
        self.slots = [torch.zeros(batch, dtype=torch.bool, pin_memory=True) for _ in range(EOS_LAG + 1)]
        self.events = [torch.cuda.Event() for _ in range(EOS_LAG + 1)]

    def finished(self, tok: torch.Tensor, step: int) -> bool:
        """Fold the newest tokens into `done`, publish them for `step`, and say whether every row was
        done EOS_LAG steps ago."""
        self.done |= torch.isin(tok, self.eos)
        i = step % len(self.slots)
        self.slots[i].copy_(self.done, non_blocking=True)
        self.events[i].record()
        if step - EOS_LAG < 1:                          # steps are counted from 1
            return False
        j = (step - EOS_LAG) % len(self.slots)
        self.events[j].synchronize()
        return bool(self.slots[j].all())

    def mask(self, tok: torch.Tensor) -> torch.Tensor:
        return torch.where(self.done, self.eos[0], tok)


class _DecodeStep:
    """One decode step of the model on static inputs (token ids, positions). mode False: always eager.
    mode True or "auto": WARMUP_STEPS eager steps on a side stream (timed), then the step is captured
    once in a HIP graph and replayed; "auto" times three replays and drops the graph unless their
    median beats the eager step by 10 % (the graph holds memory; a GPU-bound step gains nothing), and
    any mode falls back to eager steps if the capture runs out of memory."""

    def __init__(self, forward, kv, batch: int, ids_dtype: torch.dtype, device: torch.device, mode):
        self.forward, self.kv, self.mode, self.device = forward, kv, mode, device
        self.ids = torch.zeros(batch, 1, dtype=ids_dtype, device=device)
        self.pos = torch.zeros(batch, 1, dtype=torch.long, device=device)
        self.graph, self.out = None, None
        self.side = torch.cuda.Stream(device) if mode else None
        self.warm = 0
        self.eager_ms: float | None = None
        self.replay_ms: list[float] = []

    def __call__(self, tok: torch.Tensor, position: int) -> torch.Tensor:
        self.ids.copy_(tok.view(-1, 1))
        self.pos.fill_(position)
        if self.graph is not None:
            return self._replay()
        if not self.mode:
            return self.forward(self.ids, self.pos)
        if self.warm < WARMUP_STEPS:
            return self._warm_up()
        if self._capture():
            return self._replay()
        return self.forward(self.ids, self.pos)

    def _warm_up(self) -> torch.Tensor:
        main = torch.cuda.current_stream(self.device)
        torch.cuda.synchronize(self.device)
        t0 = time.perf_counter()
        self.side.wait_stream(main)
        with torch.cuda.stream(self.side):
            logits = self.forward(self.ids, self.pos)
        main.wait_stream(self.side)
        torch.cuda.synchronize(self.device)
        self.eager_ms = (time.perf_counter() - t0) * 1e3
        self.warm += 1
        return logits

    def _capture(self) -> bool:
        saved = self.kv.lengths()               # the capture records the step; it does not run it
        graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(graph):
                self.out = self.forward(self.ids, self.pos)
            self.graph = graph
        except torch.OutOfMemoryError:
            self.graph = self.out = None
            self.mode = False
            torch.cuda.empty_cache()
        finally:
            self.kv.set_lengths(saved)
        return self.graph is not None

    def _replay(self) -> torch.Tensor:
        timed = self.mode == "auto" and len(self.replay_ms) < 3
        if timed:
            torch.cuda.synchronize(self.device)
            t0 = time.perf_counter()
        self.graph.replay()
        self.kv.advance(1)
        logits = self.out
        if timed:
            torch.cuda.synchronize(self.device)
            self.replay_ms.append((time.perf_counter() - t0) * 1e3)
            if len(self.replay_ms) == 3 and self.median_replay_ms() > 0.9 * self.eager_ms:
                self.graph, self.out, self.mode = None, None, False       # not worth its memory
        return logits

    def median_replay_ms(self) -> float | None:
        return sorted(self.replay_ms)[len(self.replay_ms) // 2] if self.replay_ms else None


@torch.no_grad()
def generate(model, input_ids: torch.Tensor, max_new_tokens: int, *, bits: int = 4,
             cache: KushHFCache | None = None, prefill_chunk: int = 1024, cuda_graph: bool | str = "auto",
             eos_token_id: int | list[int] | None = None, do_sample: bool = False,
             temperature: float = 1.0, top_k: int = 0, stats: dict | None = None) -> torch.Tensor:
    """[B, prompt + generated] token ids; rows that reach EOS are padded with EOS.

    Args:
        cache: an optional fresh KushHFCache (to read cache.memory() afterwards).
        prefill_chunk: prompt tokens per forward of the prefill.
        cuda_graph: replay the decode step from a HIP graph: "auto" (keep it only when its replay is
            > 10 % faster than an eager step), True (always), False (never).
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
    eos_ids = [eos_token_id] if isinstance(eos_token_id, int) else list(eos_token_id or [])
    stop = _StopSignal(torch.tensor(eos_ids, dtype=torch.long, device=dev), B, dev) if eos_ids else None

    def forward(ids, pos):
        return model(input_ids=ids, position_ids=pos, past_key_values=cache, use_cache=True,
                     logits_to_keep=1).logits[:, -1]

    t0 = time.perf_counter()
    for c0 in range(0, T0, prefill_chunk):
        if stats is not None and cache.kv is not None and cache.kv.profile is None:
            cache.kv.profile = []               # time the chunks that attend over history
        ids = input_ids[:, c0:c0 + prefill_chunk]
        logits = forward(ids, torch.arange(c0, c0 + ids.shape[1], device=dev).expand(B, -1))
    tok = _pick(logits, do_sample, temperature, top_k)
    torch.cuda.synchronize(dev)
    t1 = time.perf_counter()

    kv = cache.kv
    kv.freeze(total)                           # every page reserved, the split count fixed
    step = _DecodeStep(forward, kv, B, input_ids.dtype, dev, cuda_graph)
    out = [tok]
    for i in range(1, max_new_tokens):
        if stop is not None and stop.finished(tok, i):
            break
        tok = _pick(step(tok, T0 + i - 1), do_sample, temperature, top_k)
        if stop is not None:
            tok = stop.mask(tok)
        out.append(tok)
    torch.cuda.synchronize(dev)
    if stats is not None:
        hist = sum(a.elapsed_time(b) for a, b in kv.profile) / 1e3 if kv.profile else 0.0
        kv.profile = None
        stats.update(prefill_s=t1 - t0, prefill_history_attn_s=hist, decode_s=time.perf_counter() - t1,
                     decode_tokens=B * (len(out) - 1), graph=step.graph is not None, eager_step_ms=step.eager_ms,
                     graph_step_ms=step.median_replay_ms())
    step.graph = step.out = None
    return torch.cat([input_ids, torch.stack(out, 1)], 1)
