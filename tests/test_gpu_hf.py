"""The Hugging Face entry point on the GPU kernels (needs an MI355X): the reference's GPU tests of
the transformers integration and of its graph-replayed generate (tests/test_gpu.py:114-200), and its
CPU integration tests (tests/test_cpu.py:122-232) run here on the HIP kernels.

References run in fp32 (the tiny models are fp32 on the GPU, or an fp32 copy of a half-precision
model): torch's half-precision attention math path (batched products over transposed views) is
kept out of the tests, as out of the product."""
import copy

import pytest
import torch

import kushkash_amd as kk

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")
DEV = "cuda"


def _tiny(kind, dtype=torch.float32):
    """tests/test_cpu.py:110-119: 2 layers, 8 q / 2 kv heads, head_dim 64 (qwen2: k/v projection bias)."""
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM
    common = dict(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=4096)
    if kind == "llama":
        cfg, cls = LlamaConfig(**common, head_dim=64), LlamaForCausalLM
    else:
        cfg, cls = Qwen2Config(**{**common, "hidden_size": 512}), Qwen2ForCausalLM
    torch.manual_seed(0)
    return cls(cfg).to(DEV, dtype).eval()


def _llama(hidden, head_dim, dtype, seed=0):
    """tests/test_gpu.py:114-183: 2 layers, 8 q / 2 kv heads, vocab 512."""
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=512, hidden_size=hidden, intermediate_size=2 * hidden, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=head_dim)
    torch.manual_seed(seed)
    return LlamaForCausalLM(cfg).to(DEV, dtype).eval()


def _sdpa(model, ids, cache):
    model.set_attn_implementation("sdpa")
    try:
        return model(ids, past_key_values=cache, use_cache=True).logits
    finally:
        kk.enable(model)


@pytest.mark.parametrize("kind", ["llama", "qwen2"])
def test_hf_prefill_and_decode(kind):
    """tests/test_cpu.py:122-142 on the kernels: prefill matches DynamicCache; 40 int8 decode steps
    stay within 5 % of the largest DynamicCache logit."""
    from transformers import DynamicCache
    model = _tiny(kind)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 256, (2, 75), generator=g).to(DEV)
    with torch.no_grad():
        rc = DynamicCache(config=model.config)
        ref = _sdpa(model, ids, rc)
        kk.enable(model)
        cache = kk.KushHFCache(model.config, bits=8)
        out = model(ids, past_key_values=cache, use_cache=True).logits
        assert (out - ref).abs().max() < 1e-4
        assert cache.get_seq_length() == 75 and cache.kv.gpu
        nxt = out[:, -1:].argmax(-1)
        for _ in range(40):
            a = model(nxt, past_key_values=cache, use_cache=True).logits
            r = _sdpa(model, nxt, rc)
            assert (a - r).abs().max() < 0.05 * r.abs().max()
            nxt = r.argmax(-1)
        assert cache.get_seq_length() == 115


def test_hf_chunked_prefill_and_generate():
    """tests/test_cpu.py:145-158 on the kernels."""
    model = kk.enable(_tiny("llama"))
    ids = torch.randint(0, 256, (1, 100), generator=torch.Generator().manual_seed(2)).to(DEV)
    with torch.no_grad():
        cache = kk.KushHFCache(model.config, bits=8)
        model(ids[:, :60], past_key_values=cache, use_cache=True)
        b = model(ids[:, 60:], past_key_values=cache, use_cache=True).logits     # chunk over history
        model.set_attn_implementation("sdpa")
        full = model(ids, use_cache=False).logits[:, 60:]
        kk.enable(model)
        assert (b - full).abs().max() < 0.05 * full.abs().max()
        gen = model.generate(ids, past_key_values=kk.KushHFCache(model.config, bits=4), max_new_tokens=20,
                             do_sample=False)
        assert gen.shape == (1, 120)


@pytest.mark.parametrize("kind", ["llama", "qwen2"])
def test_generate_matches_hf_generate(kind):
    """tests/test_cpu.py:188-196 on the kernels: kushkash_amd.generate (decode step replayed from a HIP
    graph) gives model.generate's tokens on the same cache type."""
    model = kk.enable(_tiny(kind))
    ids = torch.randint(0, 256, (2, 90), generator=torch.Generator().manual_seed(3)).to(DEV)
    with torch.no_grad():
        ref = model.generate(ids, past_key_values=kk.KushHFCache(model.config, bits=8), max_new_tokens=25,
                             do_sample=False)
    stats = {}
    got = kk.generate(model, ids, 25, bits=8, cuda_graph=True, stats=stats)
    assert stats["graph"] and stats["decode_tokens"] == 2 * 24
    assert torch.equal(got, ref)
    got = kk.generate(model, ids, 10, bits=4, prefill_chunk=40, eos_token_id=int(ref[0, 92]))
    assert got.shape[0] == 2 and got.shape[1] <= 100


def test_reused_cache():
    """tests/test_cpu.py:212-232 on the kernels."""
    model = kk.enable(_tiny("llama"))
    g = torch.Generator().manual_seed(4)
    p, turn = torch.randint(1, 256, (1, 20), generator=g).to(DEV), torch.randint(1, 256, (1, 10), generator=g).to(DEV)
    kw = dict(max_new_tokens=6, do_sample=False)
    with torch.no_grad():
        cache = kk.KushHFCache(model.config, bits=8)
        first = model.generate(p, past_key_values=cache, **kw)
        with pytest.raises(RuntimeError, match="holds 25 tokens"):
            model.generate(p, past_key_values=cache, **kw)
        assert cache.get_seq_length() == 25
        nxt = model.generate(torch.cat([first, turn], 1), past_key_values=cache, **kw)
        assert nxt.shape == (1, 26 + 10 + 6)
        with pytest.raises(RuntimeError, match="KushHFCache"):
            kk.generate(model, p, 4, cache=cache)
        cache.reset()
        assert torch.equal(model.generate(p, past_key_values=cache, **kw), first)
        cache.reset()
        model(p, position_ids=torch.arange(5, 25, device=DEV)[None], past_key_values=cache, use_cache=True)
        assert cache.get_seq_length() == 20


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_hf_generate_half(dtype):
    """tests/test_gpu.py:114-138 (head_dim 128): a half-precision model on an int8 cache against an fp32
    copy of it on DynamicCache: prefill logits and one decode step within 5 % of the largest logit,
    and model.generate runs."""
    from transformers import DynamicCache
    model = _llama(1024, 128, dtype)
    ref_model = copy.deepcopy(model).float()
    ids = torch.randint(0, 512, (2, 300), generator=torch.Generator().manual_seed(5)).to(DEV)
    with torch.no_grad():
        kk.enable(model)
        cache = kk.KushHFCache(model.config, bits=8)
        a0 = model(ids, past_key_values=cache, use_cache=True).logits.float()
        a1 = model(ids[:, -1:], past_key_values=cache, use_cache=True).logits.float()
        rc = DynamicCache(config=ref_model.config)
        ref_model.set_attn_implementation("sdpa")
        r0 = ref_model(ids, past_key_values=rc, use_cache=True).logits
        r1 = ref_model(ids[:, -1:], past_key_values=rc, use_cache=True).logits
        assert (a0 - r0).abs().max() < 0.05 * r0.abs().max()
        assert (a1 - r1).abs().max() < 0.05 * r1.abs().max()
        got = model.generate(ids, past_key_values=kk.KushHFCache(model.config, bits=8), max_new_tokens=32,
                             do_sample=False)
    assert got.shape == (2, 332) and torch.equal(got[:, :300], ids)


def test_generate_hip_graph():
    """tests/test_gpu.py:156-166: the graph-replayed decode gives the eager run's tokens (the same
    kernels; 79 replays, each checked through the tokens it feeds the next)."""
    model = _llama(1024, 128, torch.float16)
    ids = torch.randint(0, 512, (2, 300), generator=torch.Generator().manual_seed(6)).to(DEV)
    eager = kk.generate(model, ids, 80, bits=4, cuda_graph=False)
    stats = {}
    graphed = kk.generate(model, ids, 80, bits=4, cuda_graph=True, stats=stats)
    assert stats["graph"] and torch.equal(eager, graphed)


def test_generate_graph_auto_reports():
    """tests/test_gpu.py:169-180: chunked prefill (3 chunks, two over history) and the "auto" graph
    policy's report."""
    model = _llama(512, 64, torch.float16)
    ids = torch.randint(0, 512, (1, 2100), generator=torch.Generator().manual_seed(7)).to(DEV)
    st = {}
    out = kk.generate(model, ids, 20, bits=4, prefill_chunk=1000, stats=st)
    assert out.shape == (1, 2120)
    assert st["eager_step_ms"] is not None and st["prefill_history_attn_s"] > 0
    assert st["graph"] == (st["graph_step_ms"] is not None and st["graph_step_ms"] <= 0.9 * st["eager_step_ms"])


@pytest.mark.parametrize("graph", [False, True])
def test_generate_eos_async_stop(graph):
    """tests/test_gpu.py:183-200: tokens match the run without EOS up to the first EOS, everything after
    it is EOS, and generation stops at most 2 EOS_LAG steps after it."""
    from kushkash_amd._generate import EOS_LAG
    model = _llama(512, 64, torch.float16)
    ids = torch.randint(0, 512, (1, 100), generator=torch.Generator().manual_seed(8)).to(DEV)
    ref = kk.generate(model, ids, 60, bits=4, cuda_graph=graph)
    eos = int(ref[0, 100 + 10])
    k = next(i for i in range(100, 160) if int(ref[0, i]) == eos)
    out = kk.generate(model, ids, 60, bits=4, cuda_graph=graph, eos_token_id=eos)
    assert torch.equal(out[:, :k + 1], ref[:, :k + 1])
    assert bool((out[0, k + 1:] == eos).all())
    assert out.shape[1] <= k + 2 * EOS_LAG < ref.shape[1]


def test_generate_rotate_in_kernels():
    """An int4 cache whose rotation is folded into the kernels decodes like the same cache rotated by the
    reference's GEMM (the two rotations differ only in rounding: within 2 % of the largest logit, far
    inside int4's own error), both stay within 10 % of an fp32 DynamicCache run (int4), and
    graph-replayed generate gives the eager tokens."""
    from transformers import DynamicCache
    model = _llama(512, 128, torch.float16)
    ref_model = copy.deepcopy(model).float()
    ids = torch.randint(0, 512, (2, 200), generator=torch.Generator().manual_seed(9)).to(DEV)
    logits = {}
    with torch.no_grad():
        kk.enable(model)
        for folded in (False, True):
            cache = kk.KushHFCache(model.config, bits=4, rotate=True, rotate_in_kernels=folded)
            model(ids, past_key_values=cache, use_cache=True)
            logits[folded] = model(ids[:, -1:], past_key_values=cache, use_cache=True).logits.float()
            assert cache.kv.krot == folded
        rc = DynamicCache(config=ref_model.config)
        ref_model.set_attn_implementation("sdpa")
        ref_model(ids, past_key_values=rc, use_cache=True)
        r1 = ref_model(ids[:, -1:], past_key_values=rc, use_cache=True).logits
    top = logits[False].abs().max()
    assert (logits[True] - logits[False]).abs().max() < 0.02 * top
    for folded in (False, True):
        assert (logits[folded] - r1).abs().max() < 0.10 * r1.abs().max()
    mk = lambda: kk.KushHFCache(model.config, bits=4, max_length=260, rotate_in_kernels=True)
    eager = kk.generate(model, ids, 40, cache=mk(), cuda_graph=False)
    graphed = kk.generate(model, ids, 40, cache=mk(), cuda_graph=True)
    assert torch.equal(eager, graphed)
