"""Decode-attention benchmark of the compressed-KV hot path on one MI355X.

Headline workload ("C2"): Qwen2.5-7B-shaped layer, 28 q heads / 4 kv
heads (GQA 7), head_dim 128, int4 records, page 32, batch 64 x exactly 4096 cached tokens, bf16 q
and output. One step = one decode-attention pass of that layer (one kernel: the split-K merge is
fused), with the inputs resident in HBM; the timed steps are launched back to back.

Synthetic data (seed 0, generated on the GPU in this order): per pool, K = N(0,1) with a per-channel
bias ~ N(0, 6^2) (sigma 6) on a seeded 10% of the channels of each kv head (13 of 128), V = N(0,1),
written through the product's own quantize-and-pack kernel (Ops.write) into pages placed by a
seeded random permutation of the physical blocks; q = N(0,1).

The 155 MB of records of one pool fit in the 256 MB Infinity Cache, so steps rotate over
--pools independent KV pools (default 4, 621 MB) and every step reads records that left the
cache.

Timing: the library calls of a step are recorded once from the product's own Ops calls (for C2 over
the allocated buffers before the records are written, so the data generation then keeps the GPU busy
up to the warm-up); --warmup steps run untimed, the last four of them launched after a host
synchronization, and exactly --steps steps are launched back to back between HIP events, followed by
a synchronization. The last warm-up step keeps the GPU busy while the start event and the first timed
launches are issued, and at ~5 us of host time per launch the host then stays ahead of the GPU, so
the window holds the steps' kernels only. --graph-replay times the reference's way instead (bench/bench_decode.py:28-51: a one-step HIP
graph replayed back to back), which on ROCm adds ~5 us of device-side overhead per replay (C2: 37.8
us per step against 32.5 launched). The default warm-up of 1,000 steps (~33 ms for C2) brings the GPU
to its steady clocks.

Prints one JSON line (the driver's contract) with "roofline" (decode kernel: algorithmic bytes /
its mean duration, from HIP events around the timed decode launches) and
"cpu_baseline" (the C restatement of the reference CPU path, oracle/, on the host cores).

--config selects the other measured configurations of the path (each prints its own JSON line; the
default, c2, is the headline):
  c1        the reference's CPU-runnable case through the KushCache API (batch 1, 8 q / 2 kv heads, D 128,
            512 tokens, int4, rotation on): pack + one decode, on the GPU, with the oracle behind the same
            API on the host cores as the CPU baseline
  c3        Llama-3.1-8B decode step, 32 q / 8 kv heads, D 128, int8, batch 128 with ragged contexts
            N_i ~ U[256, 8192] (seed 0): append of one token per sequence (pos_offset -1, the vLLM
            convention) and decode over N_i + 1 tokens, in one launch (--two-launch: append, then decode)
  c4        Qwen3-8B decode, 32 q / 8 kv heads, D 128, int4, batch 8 x 131,072 tokens (K bias sigma 4 on
            5% of channels), split-K by the Ops.splits policy (--sweep adds NS 64, 128, 256 ...)
  c4-write  the chunked-prefill write of 2,048 new tokens per sequence of that layer (8 x 2,048 tokens,
            one launch; --two-launch for the reference's two), quantize-and-pack bytes read + written
  c4-unpack the packed-prefill unpack of one sequence of that layer (131,072 history tokens = 4,096
            full pages dequantized, 2,048 new rows copied; kp / vp [133,120, 8, 128] bf16), records
            read + rows written (--rot also rotates the history back)
  c4-fwht   the Walsh-Hadamard rotation (Ops.fwht) of that group's keys in place: 133,120 tokens x 8
            kv heads = 1,064,960 rows of D 128 bf16, read and written
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, vendor figure (8 TB/s)
PAGE = 32


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed steps")
    ap.add_argument("--warmup", type=int, default=1000,
                    help="untimed steps replayed right before the timed ones (the GPU reaches its steady clocks "
                         "after some tens of ms of sustained load)")
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--hq", type=int, default=28)
    ap.add_argument("--hkv", type=int, default=4)
    ap.add_argument("--dim", type=int, default=128)
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--pools", type=int, default=4, help="independent KV pools rotated across steps")
    ap.add_argument("--dtype", default="bf16", choices=("bf16", "fp16", "fp32"),
                    help="dtype of q, K, V and the output (the headline line is bf16)")
    ap.add_argument("--splits", type=int, default=0, help="split-K factor (0: Ops.splits policy)")
    ap.add_argument("--waves", type=int, default=0, help="waves per decode workgroup (0: Ops.waves policy)")
    ap.add_argument("--sweep", default="", help="c2: comma list of splits:waves, c4: comma list of splits, "
                                                "each timed and printed as a JSON line of its own after the main one")
    ap.add_argument("--sequential", action="store_true", help="pages in order instead of a random permutation")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of the decode, run --steps device-to-device copies of MIB MiB: the plain copy "
                         "kernel of known size that scales rocprofv3's FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--rot", action="store_true",
                    help="c2 / c4-write: the Walsh-Hadamard rotation folded into the kernels (rot = 1); "
                         "c4-unpack: rotate history rows back (canonical FWHT)")
    ap.add_argument("--two-launch", action="store_true",
                    help="c4-write: the reference's two launches (mode 0, mode 1); c3: append, then decode, "
                         "instead of one fused launch")
    ap.add_argument("--config", default="c2", choices=("c1", "c2", "c3", "c4", "c4-write", "c4-unpack", "c4-fwht"),
                    help="which configuration to measure (c2: the headline line)")
    ap.add_argument("--timeline", type=int, default=0, metavar="N",
                    help="c2: run on libkushhip_timeline.so and print N launches' per-workgroup phase times by XCD "
                         "(bf16, no rotation)")
    ap.add_argument("--graph-replay", action="store_true",
                    help="time the steps as replays of one-step HIP graphs (the reference's method) instead of "
                         "recorded launches")
    ap.add_argument("--floor", default="", metavar="MODE:WAVES:DEPTH[:Z[:PW]],...",
                    help="c2: after the decode line, time the decode's streaming floor (libkushfloor.so: the same "
                         "records and block tables, no attention math) in each listed launch shape -- mode 0 the "
                         "decode's grid (sequence, kv head), mode 1 a grid (sequence, Z) over every kv head of a "
                         "page range, mode 2 a persistent grid of Z workgroups claiming chunks of 2 WAVES PW pages "
                         "of a (sequence, kv head) from a device counter (balanced across XCDs); WAVES per "
                         "workgroup; DEPTH page pairs in flight per wave (2: the decode's ring)")
    ap.add_argument("--floor-timeline", type=int, default=0, metavar="N",
                    help="with --floor: also print N launches of each floor shape by XCD (per-workgroup wall clocks)")
    ap.add_argument("--traffic", default=str(ROOT / "profiles" / "decode_c2_traffic.md"),
                    help="rocprofv3 counter summary whose 'traffic_bytes_per_launch' fills roofline.traffic")
    return ap.parse_args(argv)


def make_workload(a, dev, defer: bool = False):
    """Pools of records written by the product's write kernel, per-pool block tables, q. defer: the
    buffers are allocated (and the block tables drawn) but the records and q are written only by
    w["fill"](), with the same random draws in the same order, so the timed launches can be recorded
    first."""
    import kushkash_amd as kk
    from kushkash_amd._ops import Ops, record_bytes
    B, N, Hkv, G, D, bits = a.batch, a.ctx, a.hkv, a.hq // a.hkv, a.dim, a.bits
    dtype = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[a.dtype]
    pages = -(-N // PAGE)
    RB = record_bytes(D, bits)
    ops = Ops(torch.device(dev), D, bits, G, dtype)
    nblk = a.pools * B * pages
    cache = torch.zeros(nblk, Hkv, RB, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    perm = (torch.arange(nblk, device=dev) if a.sequential
            else torch.randperm(nblk, generator=gen, device=dev)).to(torch.int32)
    tables = [perm[i * B * pages:(i + 1) * B * pages].view(B, pages).contiguous() for i in range(a.pools)]
    tail_k = torch.zeros(B, Hkv, PAGE, D, dtype=dtype, device=dev)
    tail_idx = torch.arange(B, dtype=torch.int32, device=dev)
    seq_lens = torch.full((B,), N, dtype=torch.int32, device=dev)
    q = torch.zeros(B, a.hq, D, dtype=dtype, device=dev)
    n_bias = max(1, round(0.10 * D))
    chunk = max(1, (1 << 27) // (Hkv * N * D * 2))          # sequences per write call (~128 MB of K)

    def fill():
        for i in range(a.pools):
            bias = torch.zeros(Hkv, D, device=dev)
            for h in range(Hkv):
                ch = torch.randperm(D, generator=gen, device=dev)[:n_bias]
                bias[h, ch] = 6.0 * torch.randn(n_bias, generator=gen, device=dev)
            for s0 in range(0, B, chunk):
                s1 = min(B, s0 + chunk)
                n = s1 - s0
                k = (torch.randn(n * N, Hkv, D, generator=gen, device=dev) + bias).to(dtype)
                v = torch.randn(n * N, Hkv, D, generator=gen, device=dev).to(dtype)
                qsl = torch.arange(n + 1, dtype=torch.int32, device=dev) * N
                js = torch.arange(n, dtype=torch.int32, device=dev).repeat_interleave(pages)
                jp = torch.arange(pages, dtype=torch.int32, device=dev).repeat(n)
                ops.write(k, v, qsl, seq_lens[s0:s1], tail_idx[s0:s1], js, jp, cache,
                          tables[i][s0:s1].contiguous(), tail_k, fused=True, rot=a.rot)
                del k, v
        q.copy_(torch.randn(B, a.hq, D, generator=gen, device=dev).to(dtype))
        torch.cuda.synchronize()

    if not defer:
        fill()
    return dict(ops=ops, cache=cache, tables=tables, tail_k=tail_k, tail_idx=tail_idx, seq_lens=seq_lens, q=q,
                B=B, N=N, Hkv=Hkv, G=G, D=D, bits=bits, RB=RB, pages=pages, kk=kk, rot=a.rot, fill=fill)


def algorithmic_bytes(w) -> int:
    """Bytes the step must move at minimum (the reference's quantized_bytes / time, cache.py:242,
    bench_decode.py:129, plus q, out, block table and seq_lens): split-K scratch excluded."""
    B, Hkv, G, D = w["B"], w["Hkv"], w["G"], w["D"]
    full, tail = w["N"] // PAGE, w["N"] % PAGE
    rec = B * Hkv * (full + (1 if tail else 0)) * w["RB"]
    tail_b = B * Hkv * tail * D * 2
    qo = 2 * B * Hkv * G * D * 2
    return rec + tail_b + qo + B * w["pages"] * 4 + B * 4


def decode_step(w, ns: int, waves: int):
    """(step, out): step(i) is one C2 decode step on pool i % pools, through the product's Ops."""
    ops, B, Hkv, G, D = w["ops"], w["B"], w["Hkv"], w["G"], w["D"]
    out = torch.empty_like(w["q"])
    work = torch.empty(max(1, B * Hkv * ns * G * (D + 2)), dtype=torch.float32, device=w["q"].device)
    sm = 1.0 / math.sqrt(D)
    P = len(w["tables"])

    def step(i):
        ops.decode(w["q"], out, w["cache"], w["tables"][i % P], w["seq_lens"], w["tail_idx"], w["tail_k"], sm, ns,
                   work, waves=waves, rot=w["rot"])
    return step, out


class Launches:
    """The library calls of a step, recorded once from the product's own Ops calls -- step(i) for
    i < period, each entry point with exactly the arguments Ops computed for it -- and replayed
    straight into libkushhip.so. A loop of K steps then issues its kernel launches back to back at
    ~5 us of host time each, so from the first step on the host runs ahead of the GPU and the timed
    window holds the K steps' kernels and nothing else (a HIP graph of K steps would add its launch
    latency, 27-50 us of an idle GPU for a 20-node graph, to the window). Recording runs every step of
    the period once; a step must not allocate device memory, or its recorded pointers would dangle."""

    def __init__(self, step, period: int = 1):
        from kushkash_amd import _lib
        torch.cuda.synchronize()
        allocations = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
        recorded, real = [], _lib.call

        def record(name, *args):
            recorded[-1].append((name, args))
            real(name, *args)
        _lib.call = record
        try:
            for i in range(period):
                recorded.append([])
                step(i)
        finally:
            _lib.call = real
        torch.cuda.synchronize()
        if torch.cuda.memory_stats().get("allocation.all.allocated", 0) != allocations:
            raise RuntimeError("bench: a timed step allocates device memory; its recorded launches would dangle")
        lib = _lib.lib()
        self.calls = [[(getattr(lib, name), name, args) for name, args in step_calls] for step_calls in recorded]
        self.period = period

    def run(self, first: int, n: int) -> None:
        """Steps first .. first + n - 1."""
        calls, period = self.calls, self.period
        for i in range(first, first + n):
            for fn, name, args in calls[i % period]:
                if fn(*args) != 0:
                    raise RuntimeError(f"bench: {name} failed during the timed steps")


def time_launches(launches: Launches, steps: int, warmup: int) -> float:
    """Mean ms per step: `warmup` untimed steps, the last four of them launched after a host
    synchronization, then exactly `steps` steps between HIP events on the launch stream, and a
    synchronization. On a GPU left idle by the synchronization the start event fires at once while
    the first timed kernel is still being launched (~20 us later, per the kernel trace of a 20-step
    run: ~1 us per step); with warm-up steps still running, the event fires as they end, with the
    first timed launches already queued behind it."""
    tail = min(4, warmup)                     # warm-up steps launched after the synchronization
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    launches.run(0, warmup - tail)
    torch.cuda.synchronize()
    launches.run(warmup - tail, tail)
    a.record()
    launches.run(warmup, steps)
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def time_graph(step, steps: int, warmup: int, period: int = 1) -> float:
    """--graph-replay, the reference's method (bench/bench_decode.py:28-51): each step of the period
    captured as a HIP graph of its own, `warmup` untimed replays (the last four after a host
    synchronization, as in time_launches), then exactly `steps` replays issued back to back between
    HIP events, and a synchronization."""
    graphs = []
    for i in range(period):
        step(i)                              # eager call first (lazy init outside the capture)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(i)
        graphs.append(g)
    torch.cuda.synchronize()
    tail = min(4, warmup)                     # as time_launches: the last warm-up replays after the sync
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(warmup - tail):
        graphs[i % period].replay()
    torch.cuda.synchronize()
    for i in range(warmup - tail, warmup):
        graphs[i % period].replay()
    a.record()
    for i in range(warmup, warmup + steps):
        graphs[i % period].replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def time_steps(a, step, period: int) -> float:
    """Mean ms per step of step(i) by the selected method (recorded launches, or --graph-replay)."""
    if a.graph_replay:
        return time_graph(step, a.steps, a.warmup, period)
    return time_launches(Launches(step, period), a.steps, a.warmup)


def cpu_baseline(w, budget_s: float):
    """The oracle's decode (C restatement of the reference CPU path, fp32, one task per (sequence,
    kv head)) on the host cores, over a bounded sample of the same workload: the first S_cpu
    sequences of pool 0 (records copied to host memory). Median of up to 20 runs after 3 warm-ups."""
    from oracle import cpu_ops
    B, Hkv, G, D = w["B"], w["Hkv"], w["G"], w["D"]
    ncores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():         # the box's CPU share for this GPU
        ncores = min(ncores, int(os.environ["OMP_NUM_THREADS"]))
    cpu_ops.set_threads(ncores)
    ops = cpu_ops.OracleOps("cpu", D, w["bits"], G)
    table = w["tables"][0].cpu()
    S = B
    # size the sample: one sequence timed first, then as many as fit in the budget
    cache = w["cache"].cpu()
    tail_k = w["tail_k"].float().cpu()
    q = w["q"].float().cpu()
    sl = w["seq_lens"].cpu()
    ti = w["tail_idx"].cpu()

    def run(n):
        out = torch.empty(n, Hkv * G, D)
        t0 = time.perf_counter()
        ops.decode(q[:n].contiguous(), out, cache, table[:n].contiguous(), sl[:n].contiguous(), ti[:n].contiguous(),
                   tail_k, 1.0 / math.sqrt(D))
        return time.perf_counter() - t0

    t1 = run(min(S, max(1, ncores)))
    per_seq = t1 / min(S, max(1, ncores))
    n = int(min(S, max(1, budget_s / 4 / max(per_seq, 1e-6))))
    for _ in range(3):                                           # warm-ups
        run(n)
    reps = max(1, min(20, int(budget_s / max(per_seq * n, 1e-6))))
    times = sorted(run(n) for _ in range(reps))
    med = times[len(times) // 2]
    frac = n / S
    cpu_ops.set_threads(1)                                        # single-core figure on one sequence
    t_one = min(run(1) for _ in range(2))
    cpu_ops.set_threads(ncores)
    bytes_ = algorithmic_bytes(w) * frac
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(bytes_ / med / 1e9, 3), "unit": "GB/s", "cores": ncores, "kind": "port",
            "sample": f"{n} of {S} sequences of the same C2 workload (all {Hkv} kv heads, {w['N']} tokens each), "
                      f"median of {reps} runs after 3 warm-ups; {med * 1e6 / n:.0f} us per sequence on {ncores} "
                      f"threads, {t_one * 1e6:.0f} us per sequence on 1 thread; host CPU: {cpu_model}",
            "us_per_step_extrapolated": round(med / frac * 1e6, 1)}


_IN = {torch.float32: "float", torch.float16: "_Float16", torch.bfloat16: "kush::bf16_t"}


def _b(x) -> str:
    return "true" if x else "false"


def decode_kernel_name(D: int, bits: int, dtype, waves: int, G: int, rot: bool, ns: int = 1, chunks: int = 0) -> str:
    """The instantiation kush_decode launches, as rocprofv3 names it: the requested waves unless the
    configuration's page ring does not fit in LDS (4 KB of block ids + 4 slots per wave of one record
    each, within 160 KiB), two page streams when G <= 8, wave splits as kush_decode.hip's
    wave_splits picks them for ns splits over `chunks` (sequences x kv heads x head chunks), and the
    ring depth launch_decode picks (three page pairs per wave with KUSHKASH_AMD_RING=3 where a third
    ring array fits, else two)."""
    from kushkash_amd._ops import record_bytes
    nw = waves or 8
    while nw > 2 and 4 * nw * record_bytes(D, bits) + 4 * 1024 + 16 > 160 * 1024:
        nw //= 2
    env = os.environ.get("KUSHKASH_AMD_WAVE_SPLITS", "")
    ws = nw == 4 and ns % nw == 0 and ns >= 2 * nw and (env[:1] == "1" or (env[:1] != "0" and chunks * (ns // nw) >= 256))
    rec = record_bytes(D, bits)
    fits3 = 6 * nw * rec + 4 * 1024 + 16 <= 160 * 1024 and 4 * -(-rec // 1024) <= 63
    dep = 3 if nw == 4 and not rot and not ws and fits3 and os.environ.get("KUSHKASH_AMD_RING", "")[:1] == "3" else 2
    return f"kush::decode_kernel<{D}, {bits}, {_IN[dtype]}, {nw}, {2 if G <= 8 else 1}, {_b(rot)}, {_b(ws)}, {dep}>"


# the translation unit of each kernel family (its digest covers the unit and its headers)
UNIT = {"decode_kernel": "kush_decode_inst.hip", "write_kernel": "kush_write.hip", "append_kernel": "kush_write.hip",
        "unpack_kernel": "kush_unpack.hip", "fwht_kernel": "kush_rotate.hip"}


def source_digest(kernel: str) -> str | None:
    """Digest of the sources the loaded library built `kernel` from (kushkash_amd.build: its
    translation unit and that unit's headers)."""
    import importlib
    import re
    kbuild = importlib.import_module("kushkash_amd.build")       # the module (the package exports a build())
    unit = UNIT[re.search(r"kush::(\w+)<", kernel).group(1)]
    return kbuild.built_digest(unit) or kbuild.source_digest(unit)


def measured_traffic(path: str, workload: str, kernel: str):
    """HBM bytes per launch of a configuration's main kernel from a committed counter summary
    (FETCH_SIZE + WRITE_SIZE of the same workload, each scaled by the copy-kernel calibration), or
    None. The summary must name the same workload, the same kernel instantiation and the same
    source digest as this run's library: bytes counted on another build are never reported."""
    try:
        text = Path(path).read_text()
    except OSError:
        return None
    import re
    fields = {k: v.strip() for k, v in re.findall(r"^(workload|kernel|sources|traffic_bytes_per_launch):\s*(.+)$",
                                                   text, re.M)}
    if (fields.get("workload") != workload or fields.get("kernel") != kernel
            or fields.get("sources") != source_digest(kernel) or "traffic_bytes_per_launch" not in fields):
        return None
    return int(fields["traffic_bytes_per_launch"])


def copy_calibration(a) -> None:
    """Plain copies of a known size, for the byte counters' scale factor."""
    n = a.calibrate_copy << 20
    x = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        y.copy_(x)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / a.steps
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "copies": a.steps + 3,
                      "us_per_copy": round(dt * 1e6, 2), "GB/s": round(2 * n / dt / 1e9, 1)}), flush=True)


# ---------------------------------------------------------------- other configurations (C3, C4)
def ragged_cache(ops, lens, room: int, Hkv: int, bias_sigma: float, bias_frac: float, gen, dev):
    """One pool of records for sequences of lens[i] tokens (pages for lens[i] + room), written by the
    product's write kernel from seeded K = N(0,1) + per-channel bias (sigma bias_sigma on a seeded
    bias_frac of the channels of each kv head) and V = N(0,1); pages placed by a seeded permutation."""
    from kushkash_amd._ops import record_bytes
    D, bits, dtype = ops.D, ops.bits, ops.dtype
    B = len(lens)
    pages = [-(-(n + room) // PAGE) for n in lens]
    total, maxp = sum(pages), max(pages)
    cache = torch.zeros(total, Hkv, record_bytes(D, bits), dtype=torch.uint8, device=dev)
    perm = torch.randperm(total, generator=gen, device=dev).to(torch.int32)
    table = torch.zeros(B, maxp, dtype=torch.int32, device=dev)
    off = 0
    for i, p in enumerate(pages):
        table[i, :p] = perm[off:off + p]
        off += p
    tail_k = torch.zeros(B, Hkv, PAGE, D, dtype=dtype, device=dev)
    tail_idx = torch.arange(B, dtype=torch.int32, device=dev)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    n_bias = max(1, round(bias_frac * D))
    bias = torch.zeros(Hkv, D, device=dev)
    for h in range(Hkv):
        ch = torch.randperm(D, generator=gen, device=dev)[:n_bias]
        bias[h, ch] = bias_sigma * torch.randn(n_bias, generator=gen, device=dev)
    s0 = 0
    while s0 < B:                            # ~2^27 K elements per write call
        s1, n_tok = s0, 0
        while s1 < B and (s1 == s0 or n_tok + lens[s1] <= (1 << 27) // (Hkv * D)):
            n_tok += lens[s1]
            s1 += 1
        k = (torch.randn(n_tok, Hkv, D, generator=gen, device=dev) + bias).to(dtype)
        v = torch.randn(n_tok, Hkv, D, generator=gen, device=dev).to(dtype)
        ln = lens[s0:s1]
        qsl = torch.tensor([0] + list(torch.tensor(ln).cumsum(0)), dtype=torch.int32, device=dev)
        js = torch.cat([torch.full((-(-n // PAGE),), i, dtype=torch.int32) for i, n in enumerate(ln)]).to(dev)
        jp = torch.cat([torch.arange(-(-n // PAGE), dtype=torch.int32) for n in ln]).to(dev)
        ops.write(k, v, qsl, seq_lens[s0:s1], tail_idx[s0:s1], js, jp, cache, table[s0:s1].contiguous(), tail_k,
                  fused=True)
        del k, v
        s0 = s1
    torch.cuda.synchronize()
    return cache, table, tail_k, tail_idx


def _line(metric, us, alg, config, kernel, extra=None, traffic_md=None):
    """One JSON line for a configuration; `kernel` is the main kernel's instantiation (rocprofv3's name)."""
    gbs = alg / (us * 1e-6) / 1e9
    traffic = measured_traffic(str(ROOT / "profiles" / traffic_md), config["workload"], kernel) if traffic_md else None
    res = {"metric": metric, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "us_per_step": round(us, 2),
           "pct_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 1), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "data": "synthetic (seeded, generated on the GPU)", "config": config,
           "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "kernel": kernel,
                        "sources": source_digest(kernel), "algorithmic_bytes": int(alg)}}
    if extra:
        res.update(extra)
    print(json.dumps(res), flush=True)


def bench_c1(a) -> None:
    """C1, the reference's CPU-runnable case, through the KushCache API: batch 1, 8 q / 2 kv heads,
    D 128, page 32, a 512-token context, int4 (rotation on: the default for 4-bit), bf16 K, V, q ~
    N(0,1) from seed 0 (CPU generator, in that order). One step = pack the context (write) + one decode
    step (attend) on a reset cache. The GPU line runs the product; the CPU baseline runs the same API
    calls on the oracle (the C restatement of the reference's CPU path, fp32, as the reference's CPU
    cache converts its inputs) on the host cores, all threads and one. Each side: median wall time of
    20 steps after 3 warm-ups, synchronized around each step."""
    import kushkash_amd as kk
    from kushkash_amd import cache as cache_mod
    from kushkash_amd._ops import record_bytes
    from oracle import cpu_ops
    B, Hq, Hkv, D, N, bits = 1, 8, 2, 128, 512, 4
    g = torch.Generator().manual_seed(0)
    K = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16)
    V = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)

    def timed(step, sync):
        for _ in range(3):
            step()
        times = []
        for _ in range(20):
            sync()
            t0 = time.perf_counter()
            step()
            sync()
            times.append(time.perf_counter() - t0)
        return sorted(times)[len(times) // 2]

    gpu = kk.KushCache(1, Hkv, Hq, D, batch_size=B, bits=bits, device="cuda", dtype=torch.bfloat16)
    Kd, Vd, qd = K.cuda(), V.cuda(), q.cuda()

    def gpu_step():
        gpu.reset()
        gpu.write(0, Kd, Vd)
        gpu.attend(0, qd)

    t_gpu = timed(gpu_step, torch.cuda.synchronize)
    real = cache_mod.Ops
    cache_mod.Ops = cpu_ops.OracleOps                 # the CPU baseline leg only: the oracle behind the API
    try:
        cpu = kk.KushCache(1, Hkv, Hq, D, batch_size=B, bits=bits, device="cpu", dtype=torch.float32)
    finally:
        cache_mod.Ops = real
    Kc, Vc, qc = K.float(), V.float(), q.float()

    def cpu_step():
        cpu.reset()
        cpu.write(0, Kc, Vc)
        cpu.attend(0, qc)

    ncores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        ncores = min(ncores, int(os.environ["OMP_NUM_THREADS"]))
    cpu_ops.set_threads(ncores)
    torch.set_num_threads(ncores)
    t_cpu = timed(cpu_step, lambda: None)
    cpu_ops.set_threads(1)
    torch.set_num_threads(1)
    t_cpu1 = timed(cpu_step, lambda: None)
    cpu_ops.set_threads(ncores)
    torch.set_num_threads(ncores)
    RB = record_bytes(D, bits)
    recs = B * Hkv * (N // PAGE) * RB
    alg = 2 * B * Hkv * N * D * 2 + 2 * recs + 2 * B * Hq * D * 2      # K, V in; records out, read back; q, out
    cpu_model = next((l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")), "")
    _line("C1 pack + decode us/step (KushCache API), int4, 1 x 512 ctx", t_gpu * 1e6, alg,
          {"workload": f"C1 KushCache API: {Hq} q / {Hkv} kv heads, D {D}, int{bits}, page 32, batch {B} x {N} "
                       f"tokens, rotation on: write(512 tokens) + attend", "global_batch": B, "seq_len": N},
          decode_kernel_name(D, bits, torch.bfloat16, gpu.ops.waves(B, Hkv, 1, N // PAGE), Hq // Hkv, False),
          extra={"cpu_baseline": {"value": round(alg / t_cpu / 1e9, 4), "unit": "GB/s", "cores": ncores,
                                  "kind": "port", "us_per_step": round(t_cpu * 1e6, 1),
                                  "us_per_step_1_thread": round(t_cpu1 * 1e6, 1),
                                  "sample": f"the whole C1 step (write + attend through the KushCache API on the "
                                            f"oracle, fp32), median of 20 after 3 warm-ups, {ncores} threads and 1; "
                                            f"host CPU: {cpu_model}"},
                 "timing": "wall clock, eager API calls, synchronized around each step"})


def bench_c3(a) -> None:
    """C3: Llama-3.1-8B, int8, batch 128, ragged N_i ~ U[256, 8192]; one step = append + decode."""
    from kushkash_amd._ops import Ops, record_bytes
    dev = "cuda:0"
    B, Hq, Hkv, D, bits = 128, 32, 8, 128, 8
    G, dtype = Hq // Hkv, torch.bfloat16
    lens = torch.randint(256, 8193, (B,), generator=torch.Generator().manual_seed(0)).tolist()
    ops = Ops(torch.device(dev), D, bits, G, dtype)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    cache, table, tail_k, tail_idx = ragged_cache(ops, lens, 1, Hkv, 6.0, 0.10, gen, dev)
    k_new = torch.randn(B, Hkv, D, generator=gen, device=dev).to(dtype)
    v_new = torch.randn(B, Hkv, D, generator=gen, device=dev).to(dtype)
    q = torch.randn(B, Hq, D, generator=gen, device=dev).to(dtype)
    out = torch.empty_like(q)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev) + 1        # counts the appended token
    ns = a.splits or ops.splits(B, Hkv, max(n + 1 for n in lens) // PAGE)
    work = torch.empty(max(1, B * Hkv * ns * G * (D + 2)), dtype=torch.float32, device=dev)
    sm = 1.0 / math.sqrt(D)

    # longest sequences first (from the host-side lengths, as a serving engine's metadata builder has
    # them): the ragged batch's long workgroups start first
    order = torch.tensor(sorted(range(B), key=lambda i: -lens[i]), dtype=torch.int32, device=dev)
    wv = a.waves or ops.waves(B, Hkv, ns, max(n1 for n1 in lens) // PAGE + 1)

    def step(i):
        if a.two_launch:                          # the reference's pair of launches
            ops.append(k_new, v_new, sl, tail_idx, cache, table, tail_k, pos_offset=-1, advance=False)
            ops.decode(q, out, cache, table, sl, tail_idx, tail_k, sm, ns, work, waves=wv, order=order)
        else:                                     # one launch: the page's workgroup appends first
            ops.append_decode(k_new, v_new, q, out, cache, table, sl, tail_idx, tail_k, sm, ns, work, waves=wv,
                              order=order)

    ms = time_steps(a, step, 1)
    RB, DC = record_bytes(D, bits), (D if bits == 8 else D // 2)
    n1 = [n + 1 for n in lens]
    dec = sum((n // PAGE) * Hkv * RB + (n % PAGE) * Hkv * (2 * D + DC + 4) for n in n1)
    qo = 2 * B * Hq * D * 2
    app = B * Hkv * (2 * 2 * D + DC + 4 + 2 * D)                         # k, v rows in; V row, K tail row out
    app += sum(Hkv * ((PAGE - 1) * 2 * D + PAGE * DC + 4 * D) for n in lens if n % PAGE == PAGE - 1)
    alg = dec + qo + app + B * 4 * (table.shape[1] + 2)
    _line("append + decode us/step + achieved HBM GB/s (% peak), int8, bs128 ragged U[256, 8192]", ms * 1e3, alg,
          {"workload": f"C3 Llama-3.1-8B layer: {Hq} q / {Hkv} kv heads, D {D}, int{bits}, page 32, batch {B}, "
                       f"N_i ~ U[256, 8192] (seed 0; sum {sum(lens)} tokens), append (pos_offset -1) + decode"
                       + (" (two launches)" if a.two_launch else " (one launch)"),
           "global_batch": B, "split_k": ns, "tokens": sum(n1), "sequence_order": "longest first",
           "waves": wv},
          decode_kernel_name(D, bits, dtype, wv, G, False), traffic_md="decode_c3_traffic.md",
          extra={"launches": ("append_kernel, then decode_kernel" if a.two_launch
                              else "decode_kernel with the append inside")})


def bench_c4(a) -> None:
    """C4 decode: Qwen3-8B, int4, batch 8 x 131,072 tokens, split-K."""
    from kushkash_amd._ops import Ops, record_bytes
    dev = "cuda:0"
    B, Hq, Hkv, D, bits, N = 8, 32, 8, 128, 4, 131072
    G, dtype = Hq // Hkv, torch.bfloat16
    ops = Ops(torch.device(dev), D, bits, G, dtype)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    cache, table, tail_k, tail_idx = ragged_cache(ops, [N] * B, 0, Hkv, 4.0, 0.05, gen, dev)
    q = torch.randn(B, Hq, D, generator=gen, device=dev).to(dtype)
    out = torch.empty_like(q)
    sl = torch.full((B,), N, dtype=torch.int32, device=dev)
    sm = 1.0 / math.sqrt(D)
    alg = B * Hkv * (N // PAGE) * record_bytes(D, bits) + 2 * B * Hq * D * 2 + B * 4 * (N // PAGE + 1)
    policy = ops.splits(B, Hkv, N // PAGE)
    nss = [a.splits or policy] + [int(x) for x in a.sweep.split(",") if x.strip() and ":" not in x]
    for i, ns in enumerate(nss):
        work = torch.empty(B * Hkv * ns * G * (D + 2), dtype=torch.float32, device=dev)
        wv = a.waves or ops.waves(B, Hkv, ns, N // PAGE)
        ms = time_steps(a, lambda j: ops.decode(q, out, cache, table, sl, tail_idx, tail_k, sm, ns, work, waves=wv),
                        1)
        _line("decode-attn us/step + achieved HBM GB/s (% peak), int4, bs8 x 131k ctx", ms * 1e3, alg,
              {"workload": f"C4 Qwen3-8B layer: {Hq} q / {Hkv} kv heads, D {D}, int{bits}, page 32, "
                           f"batch {B} x {N} tokens, splits {ns}, waves {wv}", "global_batch": B, "seq_len": N,
               "split_k": ns, "waves": wv, "split_k_policy": ns == policy},
              decode_kernel_name(D, bits, dtype, wv, G, False, ns, B * Hkv * -(-G // 16)),
              traffic_md="decode_c4_traffic.md", extra={"merge": "split-K partials merged inside the launch"})


def bench_c4_write(a) -> None:
    """C4 chunked-prefill write: 2,048 new tokens for each of 8 sequences (fresh pages), 4 rotated
    input / record sets (344 MB) so that the step reads and writes HBM, not the Infinity Cache."""
    from kushkash_amd._ops import Ops, record_bytes
    dev = "cuda:0"
    B, Hq, Hkv, D, bits, T, P = 8, 32, 8, 128, 4, 2048, 4
    G, dtype = Hq // Hkv, torch.bfloat16
    ops = Ops(torch.device(dev), D, bits, G, dtype)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    pages = T // PAGE
    RB = record_bytes(D, bits)
    sets = []
    for p in range(P):
        cache = torch.zeros(B * pages, Hkv, RB, dtype=torch.uint8, device=dev)
        table = torch.randperm(B * pages, generator=gen, device=dev).to(torch.int32).view(B, pages).contiguous()
        k = torch.randn(B * T, Hkv, D, generator=gen, device=dev).to(dtype)
        v = torch.randn(B * T, Hkv, D, generator=gen, device=dev).to(dtype)
        sets.append((k, v, cache, table))
    tail_k = torch.zeros(B, Hkv, PAGE, D, dtype=dtype, device=dev)
    tail_idx = torch.arange(B, dtype=torch.int32, device=dev)
    sl = torch.full((B,), T, dtype=torch.int32, device=dev)
    qsl = torch.arange(B + 1, dtype=torch.int32, device=dev) * T
    js = torch.arange(B, dtype=torch.int32, device=dev).repeat_interleave(pages)
    jp = torch.arange(pages, dtype=torch.int32, device=dev).repeat(B)

    def step(i):
        k, v, cache, table = sets[i % P]
        ops.write(k, v, qsl, sl, tail_idx, js, jp, cache, table, tail_k, fused=not a.two_launch, rot=a.rot)

    ms = time_steps(a, step, P)
    alg = 2 * B * T * Hkv * D * 2 + B * pages * Hkv * RB
    launches = ("two launches: mode 0, mode 1" if a.two_launch else "one launch: mode 2") + (", rot" if a.rot else "")
    _line("chunked-prefill write us/step + achieved HBM GB/s (% peak), int4, 8 x 2048 tokens", ms * 1e3, alg,
          {"workload": f"C4 write: {B} x {T} new tokens, {Hkv} kv heads, D {D}, int{bits} (512 page jobs x {Hkv} "
                       f"heads, {launches})", "global_batch": B, "tokens": B * T},
          f"kush::write_kernel<{D}, {bits}, kush::bf16_t, true, {_b(not a.two_launch)}, {_b(a.rot)}>",
          traffic_md="write_c4_traffic.md", extra={"launches": launches})


def bench_c4_unpack(a) -> None:
    """C4 packed-prefill unpack: the group of one sequence, [4,096 history pages | 2,048 new rows], as
    the vLLM backend builds it before flash-attn (kushkash/vllm/backend.py:837-856). Two record pools
    (310 MB) alternate across steps; kp / vp (545 MB) are rewritten every step."""
    from kushkash_amd._ops import Ops, record_bytes
    dev = "cuda:0"
    Hkv, D, bits, N, T, P = 8, 128, 4, 131072, 2048, 2
    dtype = torch.bfloat16
    ops = Ops(torch.device(dev), D, bits, 1, dtype)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    pools = [ragged_cache(ops, [N], 0, Hkv, 4.0, 0.05, gen, dev) for _ in range(P)]
    pages = N // PAGE
    rows = N + T
    page_dst = torch.arange(pages, dtype=torch.int32, device=dev) * PAGE
    new_dst = torch.arange(N, rows, dtype=torch.int32, device=dev)
    none = torch.zeros(0, dtype=torch.int32, device=dev)
    k_new = torch.randn(T, Hkv, D, generator=gen, device=dev).to(dtype)
    v_new = torch.randn(T, Hkv, D, generator=gen, device=dev).to(dtype)
    kp = torch.empty(rows, Hkv, D, dtype=dtype, device=dev)
    vp = torch.empty_like(kp)
    blks = [p[1][0, :pages].contiguous() for p in pools]

    def step(i):
        cache, _, tail_k, _ = pools[i % P]
        ops.unpack(cache, blks[i % P], page_dst, none, none, tail_k, k_new, v_new, new_dst, kp, vp, a.rot)

    ops.validate = True                        # indices checked once, outside the timed steps
    step(0)
    ops.validate = False
    ms = time_steps(a, step, P)
    RB = record_bytes(D, bits)
    alg = pages * Hkv * RB + 2 * rows * Hkv * D * 2 + 2 * T * Hkv * D * 2
    extra = None
    if not a.no_cpu_baseline:
        extra = {"cpu_baseline": cpu_baseline_unpack(pools[0], blks[0], k_new, v_new, D, bits, Hkv, a.rot,
                                                     min(a.cpu_seconds, 10.0))}
    _line("prefill-unpack us/step + achieved HBM GB/s (% peak), int4, 131k history + 2048 new", ms * 1e3, alg,
          {"workload": f"C4 packed-prefill unpack: 1 x ({N} history + {T} new) tokens, {Hkv} kv heads, D {D}, "
                       f"int{bits}, bf16 kp / vp, rot {int(a.rot)}", "global_batch": 1, "seq_len": rows},
          f"kush::unpack_kernel<{D}, {bits}, kush::bf16_t, true>", extra, traffic_md="unpack_c4_traffic.md")


def cpu_baseline_unpack(pool, blk, k_new, v_new, D, bits, Hkv, rot, budget_s: float):
    """The oracle's unpack (C restatement of the reference CPU kernel, fp32, one thread) over a
    bounded sample of the same group: its first n history pages, no new rows."""
    from kushkash_amd._ops import record_bytes
    from oracle import cpu_ops
    cache, _, tail_k, _ = pool
    ops = cpu_ops.OracleOps("cpu", D, bits, 1)
    cache_h, blk_h = cache.cpu(), blk.cpu()
    tail_h = tail_k.float().cpu()
    none = torch.zeros(0, dtype=torch.int32)
    empty = torch.zeros(0, Hkv, D)

    def run(n):
        kp = torch.empty(n * PAGE, Hkv, D)
        vp = torch.empty_like(kp)
        dst = torch.arange(n, dtype=torch.int32) * PAGE
        t0 = time.perf_counter()
        ops.unpack(cache_h, blk_h[:n].contiguous(), dst, none, none, tail_h, empty, empty, none, kp, vp, rot)
        return time.perf_counter() - t0

    per_page = run(16) / 16
    n = int(min(blk_h.numel(), max(16, budget_s / 4 / max(per_page, 1e-9))))
    for _ in range(3):
        run(n)
    reps = max(1, min(10, int(budget_s / max(per_page * n, 1e-9))))
    med = sorted(run(n) for _ in range(reps))[reps // 2]
    alg = n * Hkv * record_bytes(D, bits) + 2 * n * PAGE * Hkv * D * 4
    return {"value": round(alg / med / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n} of {blk_h.numel()} history pages of the same group (all {Hkv} kv heads, fp32 kp / vp, "
                      f"rot {int(rot)}), median of {reps} runs after 3 warm-ups; {med * 1e6 / n:.1f} us per page"}


def bench_c4_fwht(a) -> None:
    """Ops.fwht over one C4 packed group's keys, in place (two alternating 272 MB buffers)."""
    from kushkash_amd._ops import Ops
    dev = "cuda:0"
    Hkv, D, rows = 8, 128, 131072 + 2048
    dtype = torch.bfloat16
    ops = Ops(torch.device(dev), D, 4, 1, dtype)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    xs = [torch.randn(rows * Hkv, D, generator=gen, device=dev).to(dtype) for _ in range(2)]
    ms = time_steps(a, lambda i: ops.fwht(xs[i % 2], out=xs[i % 2]), 2)
    alg = 2 * rows * Hkv * D * 2
    _line("fwht us/step + achieved HBM GB/s (% peak), 1,064,960 rows of D 128 bf16", ms * 1e3, alg,
          {"workload": f"C4 key rotation: {rows} tokens x {Hkv} kv heads, D {D}, bf16, in place", "rows": rows * Hkv},
          f"kush::fwht_kernel<{D}, kush::bf16_t, true>", traffic_md="fwht_c4_traffic.md")


def bench_timeline(a) -> None:
    """C2 decode on the timeline build (kushkash_amd/libkushhip_timeline.so: the same kernels, wave 0 of
    each workgroup timestamping five phases and each wave its pages done, kush_decode.h KUSH_TIMELINE):
    after `--warmup` eager steps per probed launch, one launch is recorded and summarized as markdown --
    each phase's spread over the workgroups (us from the first workgroup's start), how far apart the
    waves of a workgroup finish their pages, and per XCD the page-loop time (first pair landed -> pages
    done), the pages-done times and the shader clock over the loop."""
    import ctypes
    import importlib
    import numpy as np
    from kushkash_amd import _lib
    kbuild = importlib.import_module("kushkash_amd.build")
    if a.dtype != "bf16" or a.rot:
        raise SystemExit("--timeline: the timeline build instruments the bf16, unrotated decode only")
    if not kbuild.TIMELINE_LIB.exists():
        raise SystemExit(f"--timeline: {kbuild.TIMELINE_LIB.name} is not built; run `python -m kushkash_amd.build`")
    _lib.LIB = kbuild.TIMELINE_LIB
    _lib.lib.cache_clear()
    read = _lib.lib().kush_timeline_read
    read.argtypes, read.restype = [ctypes.c_void_p, ctypes.c_int64], ctypes.c_int32
    w = make_workload(a, "cuda:0")
    ops, B, Hkv, G, D = w["ops"], w["B"], w["Hkv"], w["G"], w["D"]
    ns = a.splits or ops.splits(B, Hkv, w["N"] // PAGE)
    wv = a.waves or ops.waves(B, Hkv, ns, w["pages"])
    kernel = decode_kernel_name(a.dim, a.bits, ops.dtype, wv, G, False, ns, B * Hkv * -(-G // 16))
    out = torch.empty_like(w["q"])
    work = torch.empty(max(1, B * Hkv * ns * G * (D + 2)), dtype=torch.float32, device="cuda:0")
    sm = 1.0 / math.sqrt(D)

    def step(i):
        ops.decode(w["q"], out, w["cache"], w["tables"][i % len(w["tables"])], w["seq_lens"], w["tail_idx"],
                   w["tail_k"], sm, ns, work, waves=wv)

    rows = B * Hkv * ns                       # workgroups of the launch (G <= 16: one head chunk)
    print(f"workload: C2 decode layer, {a.hq} q / {a.hkv} kv heads, D {a.dim}, int{a.bits}, batch {B} x {a.ctx} "
          f"tokens, splits {ns}, waves {wv}\nkernel: {kernel}\nsources: {source_digest(kernel)}\n"
          f"clocks: wall 100 MHz (s_memrealtime), shader clock (s_memtime); {rows} workgroups", flush=True)
    for rep in range(a.timeline):
        for i in range(a.warmup):
            step(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        step(1)
        e1.record()
        torch.cuda.synchronize()
        buf = np.zeros((rows, 16), dtype=np.int64)
        rc = read(buf.ctypes.data_as(ctypes.c_void_p), rows)
        if rc != 0:
            raise RuntimeError(f"kush_timeline_read failed ({rc})")
        t = buf.astype(np.float64)
        us = (t[:, :5] - t[:, 0].min()) / 100.0
        loop = us[:, 3] - us[:, 2]
        mhz = (t[:, 6] - t[:, 5]) / np.maximum(loop, 1e-3)
        xcd = t[:, 7].astype(int)
        pct = lambda x, p: float(np.percentile(x, p))
        print(f"\nlaunch {rep + 1} of {a.timeline}: HIP-event time {e0.elapsed_time(e1) * 1e3:.2f} us, first "
              f"workgroup start -> last output stored {us[:, 4].max():.2f} us\n\n"
              "| phase (us from the first start) | min | p10 | p50 | p90 | max |\n|---|---|---|---|---|---|")
        for name, k in (("start", 0), ("prologue done", 1), ("first page pair landed", 2), ("pages done", 3),
                        ("output stored", 4)):
            x = us[:, k]
            print(f"| {name} | {x.min():.2f} | {pct(x, 10):.2f} | {pct(x, 50):.2f} | {pct(x, 90):.2f} | {x.max():.2f} |")
        wd = (t[:, 8:8 + wv] - t[:, 0].min()) / 100.0       # every wave's pages done
        spread = wd.max(1) - wd.min(1)
        last = np.bincount(wd.argmax(1), minlength=wv)
        print(f"\nwaves' pages done within a workgroup: spread (last - first) p50 {pct(spread, 50):.2f}, p90 "
              f"{pct(spread, 90):.2f}, max {spread.max():.2f} us; mean lag behind the workgroup's first wave, by wave: "
              + ", ".join(f"{(wd[:, i] - wd.min(1)).mean():.2f}" for i in range(wv))
              + "; last to finish, by wave: " + ", ".join(str(int(c)) for c in last))
        print("\n| XCD | workgroups | page loop p10 / p50 / max (us) | pages done p50 / max (us) | "
              "shader clock p50 (MHz) |\n|---|---|---|---|---|")
        for x in range(8):
            m = xcd == x
            if m.any():
                print(f"| {x} | {int(m.sum())} | {pct(loop[m], 10):.2f} / {pct(loop[m], 50):.2f} / {loop[m].max():.2f} | "
                      f"{pct(us[m, 3], 50):.2f} / {us[m, 3].max():.2f} | {pct(mhz[m], 50):.0f} |", flush=True)


def _floor_fn(name: str = "kush_floor_stream"):
    """kush_floor_stream / kush_floor_dynamic of the measurement library (kushkash_amd/csrc/kush_floor.hip)."""
    import ctypes
    import importlib
    kbuild = importlib.import_module("kushkash_amd.build")
    if not kbuild.FLOOR_LIB.exists():
        raise SystemExit(f"--floor: {kbuild.FLOOR_LIB.name} is not built; run `python -m kushkash_amd.build`")
    fn = getattr(ctypes.CDLL(str(kbuild.FLOOR_LIB)), name)
    P, I32, I64, U32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
    if name == "kush_floor_stream":
        fn.argtypes = [I32, I32, P, I64, I64, P, P, I64, I32, I32, I32, I32, I32, I32, I32, P, P, P]
    else:
        fn.argtypes = [I32, I32, P, I64, I64, P, P, I64, I32, I32, I32, I32, I32, I32, I32, P, U32, P, P, P]
    fn.restype = I32
    return fn


class FloorLaunches:
    """The decode's streaming floor over the workload's pools, step i on pool i % pools, in one launch
    shape (mode, waves, depth, z[, pw]); run() has the interface of Launches.run, so time_launches times
    it the way it times the decode. Mode 2 (dynamic chunks) keeps one device counter, zeroed once; launch
    k passes base k x n_chunks (each launch makes exactly n_chunks claims)."""

    def __init__(self, w, mode: int, waves: int, depth: int, z: int, pw: int = 4, marks: bool = False):
        cache, B, Hkv, pages = w["cache"], w["B"], w["Hkv"], w["pages"]
        self.mode = mode
        self.wgs = B * (z if mode == 1 else Hkv) if mode != 2 else z
        self.sums = torch.empty(self.wgs * waves * 64, dtype=torch.int32, device=cache.device)
        self.marks = torch.zeros(self.wgs, 8, dtype=torch.int64, device=cache.device) if marks else None
        stream = torch.cuda.current_stream().cuda_stream
        mk = None if self.marks is None else self.marks.data_ptr()
        if mode == 2:
            self.fn = _floor_fn("kush_floor_dynamic")
            self.ctr = torch.zeros(1, dtype=torch.int32, device=cache.device)
            cp = 2 * waves * pw
            self.n_chunks = B * Hkv * ((pages + cp - 1) // cp)
            self.launches = 0
            self.args = [[w["D"], w["bits"], cache.data_ptr(), cache.stride(0), cache.stride(1), t.data_ptr(),
                          w["seq_lens"].data_ptr(), t.stride(0), Hkv, B, pages, z, waves, depth, pw,
                          self.ctr.data_ptr(), 0, self.sums.data_ptr(), mk, stream] for t in w["tables"]]
        else:
            self.fn = _floor_fn()
            self.args = [[w["D"], w["bits"], cache.data_ptr(), cache.stride(0), cache.stride(1), t.data_ptr(),
                          w["seq_lens"].data_ptr(), t.stride(0), Hkv, B, pages, mode, z, waves, depth,
                          self.sums.data_ptr(), mk, stream] for t in w["tables"]]
        self.run(0, 1)
        torch.cuda.synchronize()

    def run(self, first: int, n: int) -> None:
        for i in range(first, first + n):
            args = self.args[i % len(self.args)]
            if self.mode == 2:
                args[16] = (self.launches * self.n_chunks) & 0xFFFFFFFF
                self.launches += 1
            rc = self.fn(*args)
            if rc != 0:
                raise SystemExit(f"--floor: the floor kernel refused or failed ({rc}) for mode {self.mode}")


def floor_shapes(spec: str):
    for item in [x for x in spec.split(",") if x.strip()]:
        v = [int(x) for x in item.split(":")]
        if len(v) not in (3, 4, 5):
            raise SystemExit(f"--floor: '{item}' is not MODE:WAVES:DEPTH[:Z[:PW]]")
        yield v[0], v[1], v[2], (v[3] if len(v) >= 4 else 1), (v[4] if len(v) == 5 else 4)


def floor_timeline(w, shape, reps: int, warmup: int) -> None:
    """Per-workgroup wall clocks of one floor launch (after `warmup` untimed ones), by XCD, as markdown."""
    import numpy as np
    mode, wv, depth, z, pw = shape
    fl = FloorLaunches(w, mode, wv, depth, z, pw, marks=True)
    for rep in range(reps):
        fl.run(0, warmup)
        torch.cuda.synchronize()
        fl.run(1, 1)
        torch.cuda.synchronize()
        t = fl.marks.cpu().numpy().astype(np.float64)
        t0 = t[:, 0].min()
        us = (t[:, [0, 1, 2, 3]] - t0) / 100.0
        xcd = t[:, 4].astype(int)
        loop = us[:, 3] - us[:, 2]
        pct = lambda x, p: float(np.percentile(x, p))
        print(f"\nfloor mode {mode}, {wv} waves, depth {depth}" + (f", z {z}" if mode == 1 else "")
              + (f", {z} workgroups, chunks of {2 * wv * pw} pages" if mode == 2 else "")
              + f": launch {rep + 1} of {reps}, first workgroup start -> last pages done {us[:, 3].max():.2f} us\n\n"
              "| phase (us from the first start) | min | p10 | p50 | p90 | max |\n|---|---|---|---|---|---|")
        for name, k in (("start", 0), ("first page DMAs issued", 1), ("first page pair landed", 2), ("pages done", 3)):
            x = us[:, k]
            print(f"| {name} | {x.min():.2f} | {pct(x, 10):.2f} | {pct(x, 50):.2f} | {pct(x, 90):.2f} | {x.max():.2f} |")
        print("\n| XCD | workgroups | page loop p10 / p50 / max (us) | pages done p50 / max (us) |"
              + (" chunks |\n|---|---|---|---|---|" if mode == 2 else "\n|---|---|---|---|"))
        for x in range(8):
            m = xcd == x
            if m.any():
                print(f"| {x} | {int(m.sum())} | {pct(loop[m], 10):.2f} / {pct(loop[m], 50):.2f} / {loop[m].max():.2f} | "
                      f"{pct(us[m, 3], 50):.2f} / {us[m, 3].max():.2f} |"
                      + (f" {int(t[m, 5].sum())} |" if mode == 2 else ""), flush=True)


def main(argv=None):
    a = parse_args(argv)
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        raise SystemExit(2)
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    dev = "cuda:0"
    if a.calibrate_copy:
        copy_calibration(a)
        return
    if a.timeline:
        if a.config != "c2":
            raise SystemExit("--timeline instruments the c2 decode")
        bench_timeline(a)
        return
    if a.config != "c2":
        {"c1": bench_c1, "c3": bench_c3, "c4": bench_c4, "c4-write": bench_c4_write, "c4-unpack": bench_c4_unpack,
         "c4-fwht": bench_c4_fwht}[a.config](a)
        return
    # The steps' launches are recorded over the allocated buffers before the records are written: the
    # data generation (the write kernel over every pool) then keeps the GPU busy up to the warm-up.
    w = make_workload(a, dev, defer=True)
    ns = a.splits or w["ops"].splits(w["B"], w["Hkv"], w["N"] // PAGE)
    alg = algorithmic_bytes(w)

    wv = a.waves or w["ops"].waves(w["B"], w["Hkv"], ns, w["pages"])
    step, _ = decode_step(w, ns, wv)
    P = len(w["tables"])
    if a.graph_replay:
        w["fill"]()
        ms = time_graph(step, a.steps, a.warmup, P)
    else:
        launches = Launches(step, P)
        w["fill"]()
        ms = time_launches(launches, a.steps, a.warmup)
    shape = (f"C2 Qwen2.5-7B decode layer: {a.hq} q / {a.hkv} kv heads, D {a.dim}, int{a.bits}, page 32, "
             f"batch {a.batch} x {a.ctx} tokens" + (", rotation folded into the kernels" if a.rot else "")
             + ("" if a.dtype == "bf16" else f", {a.dtype}"))
    workload = f"{shape}, splits {ns}, waves {wv}"
    kernel = decode_kernel_name(a.dim, a.bits, w["ops"].dtype, wv, w["G"], a.rot, ns, w["B"] * w["Hkv"] * -(-w["G"] // 16))
    ms_dec = ms                                   # one kernel per step: the decode kernel is the step
    gbs = alg / ms / 1e6
    gbs_dec = alg / ms_dec / 1e6
    res = {
        "metric": "decode-attn us/step + achieved HBM GB/s (% peak), int4, bs64 x 4k ctx",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_step": round(ms * 1e3, 2),
        "pct_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 1),
        "tokens_per_s": round(w["B"] / (ms / 1e3), 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 records, f16 MFMA, f32 accumulate, bf16 q/out",
        "data": "synthetic (seeded; K bias sigma 6 on 10% of channels; random page placement; "
                f"{a.pools} rotated pools)",
        "config": {"workload": workload, "global_batch": a.batch,
                   "seq_len": a.ctx, "parallelism": "single GPU", "split_k": ns, "waves": wv, "pools": a.pools},
        "roofline": {"bound": "hbm", "achieved": round(gbs_dec, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs_dec / PEAK_HBM_GBS, 4),
                     "traffic": measured_traffic(a.traffic, workload, kernel),
                     "kernel": kernel, "sources": source_digest(kernel), "step_us": round(ms_dec * 1e3, 2),
                     "algorithmic_bytes": alg},
        "cpu_baseline": None,
    }
    if not a.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(w, a.cpu_seconds)
    print(json.dumps(res), flush=True)

    for mode, fwv, depth, z, pw in floor_shapes(a.floor):          # the streaming floor, a line each
        fms = time_launches(FloorLaunches(w, mode, fwv, depth, z, pw), a.steps, a.warmup)
        rec = w["B"] * w["Hkv"] * (w["N"] // PAGE) * w["RB"]
        kname = (f"kush_floor_stream (floor_kernel<{a.dim}, {a.bits}, {fwv}, {depth}>)" if mode != 2 else
                 f"kush_floor_dynamic (floor_dyn_kernel<{a.dim}, {a.bits}, {fwv}, {depth}, {pw}>)")
        print(json.dumps({"floor": {"mode": mode, "waves": fwv, "depth": depth, "z": z if mode else None,
                                    "chunk_pages": 2 * fwv * pw if mode == 2 else None},
                          "kernel": kname,
                          "us_per_step": round(fms * 1e3, 2), "records_GBps": round(rec / fms / 1e6, 1),
                          "pct_peak_hbm": round(100 * alg / fms / 1e6 / PEAK_HBM_GBS, 1),
                          "decode_us_per_step": round(ms * 1e3, 2)}), flush=True)
        if a.floor_timeline:
            floor_timeline(w, (mode, fwv, depth, z, pw), a.floor_timeline, min(a.warmup, 200))

    for item in [x for x in a.sweep.split(",") if x.strip()]:     # other launch shapes, a line each
        sns, swv = (int(v) for v in item.split(":"))
        msx = time_steps(a, decode_step(w, sns, swv)[0], P)
        _line(res["metric"], msx * 1e3, alg, {"workload": f"{shape}, splits {sns}, waves {swv}",
                                              "global_batch": a.batch, "seq_len": a.ctx, "split_k": sns,
                                              "waves": swv, "sweep": True},
              decode_kernel_name(a.dim, a.bits, w["ops"].dtype, swv, w["G"], a.rot, sns,
                                 w["B"] * w["Hkv"] * -(-w["G"] // 16)))


if __name__ == "__main__":
    main()
