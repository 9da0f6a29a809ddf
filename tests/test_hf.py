"""The Hugging Face entry point (kushkash_amd/hf.py) on the CPU: config checks, mask and hand-off
errors, and the reference's CPU tests of the transformers integration (tests/test_cpu.py:110-232)
with the KushCache running on the CPU oracle (the C restatement of the reference's CPU kernels) in
place of the GPU kernels, so what is tested here is hf.py's host logic. The same tests on the GPU
kernels are in test_gpu_hf.py."""
import contextlib
from types import SimpleNamespace

import pytest
import torch

import kushkash_amd as kk
from kushkash_amd import hf
from _harness import oracle_backend

transformers = pytest.importorskip("transformers")


def _tiny(kind):
    """The reference tests' tiny models (tests/test_cpu.py:110-119): 2 layers, 8 q / 2 kv heads, D 64."""
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM
    common = dict(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=4096)
    if kind == "llama":
        cfg, cls = LlamaConfig(**common, head_dim=64), LlamaForCausalLM
    else:
        cfg, cls = Qwen2Config(**{**common, "hidden_size": 512}), Qwen2ForCausalLM     # D 64, k/v bias
    torch.manual_seed(0)
    return cls(cfg).eval()


@pytest.fixture
def oracle():
    with oracle_backend():
        yield


def test_check_config_rejects_sliding_window():
    """A window that can bind is refused; one at or past max_position_embeddings never binds
    (tests/test_cpu.py:532-562)."""
    from transformers import MistralConfig, Phi3Config, Qwen2Config, Qwen2MoeConfig
    with pytest.raises(NotImplementedError, match="sliding-window"):
        hf._check_config(MistralConfig())                                   # window 4096, no layer_types
    hf._check_config(MistralConfig(sliding_window=None))
    hf._check_config(Phi3Config(sliding_window=262144, max_position_embeddings=131072))
    with pytest.raises(NotImplementedError, match="sliding-window"):
        hf._check_config(Phi3Config(sliding_window=4096, max_position_embeddings=131072))
    with pytest.raises(NotImplementedError, match="sliding-window"):
        hf._check_config(MistralConfig(layer_types=["sliding_attention"] * 32))
    with pytest.raises(NotImplementedError, match="sliding-window"):
        hf._check_config(SimpleNamespace(sliding_window=4096))              # no maximum to compare with
    with pytest.raises(NotImplementedError, match="sliding-window"):
        hf._check_config(SimpleNamespace(use_sliding_window=True))
    hf._check_config(SimpleNamespace(sliding_window=None, layer_types=["full_attention"] * 4))
    hf._check_config(Qwen2MoeConfig())
    hf._check_config(SimpleNamespace(sliding_window=1024, max_position_embeddings=131072,
                                     layer_types=["full_attention"] * 4))
    hf._check_config(Qwen2Config(sliding_window=131072, use_sliding_window=False))
    with pytest.raises(NotImplementedError, match="sliding-window"):
        hf._check_config(Qwen2Config(sliding_window=4096, use_sliding_window=True, max_window_layers=2,
                                     num_hidden_layers=4))
    hf._check_config(SimpleNamespace(sliding_window=0))


def test_check_config_rejects_softcap_and_mla():
    with pytest.raises(NotImplementedError, match="softcapping"):
        hf._check_config(SimpleNamespace(attn_logit_softcapping=50.0))
    with pytest.raises(NotImplementedError, match="MLA"):
        hf._check_config(SimpleNamespace(kv_lora_rank=512))
    with pytest.raises(NotImplementedError):
        kk.enable(SimpleNamespace(config=SimpleNamespace(use_sliding_window=True)))


def test_rejects_padding():
    """tests/test_cpu.py:161-167: a padded prompt batch is refused before any attention runs."""
    model = kk.enable(_tiny("llama"))
    ids = torch.randint(0, 256, (2, 10))
    mask = torch.ones_like(ids)
    mask[0, :3] = 0
    with pytest.raises(NotImplementedError, match="padded"):
        model(ids, attention_mask=mask, past_key_values=kk.KushHFCache(model.config), use_cache=True)


def test_forward_without_cache_raises(oracle):
    """tests/test_cpu.py:199-209: the attention function never reuses a cache of an earlier forward."""
    model = kk.enable(_tiny("llama"))
    ids = torch.randint(0, 256, (1, 10))
    with torch.no_grad():
        model(ids, past_key_values=kk.KushHFCache(model.config), use_cache=True)
        with pytest.raises(RuntimeError, match="KushHFCache"):
            model(ids, use_cache=False)


def test_cache_layer_surface():
    """What transformers reads off the layers before the first forward, and what a quantized page
    cache refuses (hf.py:34-80)."""
    model = _tiny("llama")
    c = kk.KushHFCache(model.config, bits=8)
    assert c.get_seq_length() == 0 and c.memory() is None and len(c.layers) == 2
    layer = c.layers[0]
    assert layer.get_max_length() == -1 and layer.get_mask_sizes(7) == (7, 0)
    for call in (lambda: layer.crop(3), lambda: layer.reorder_cache(torch.tensor([0])),
                 lambda: layer.batch_repeat_interleave(2), lambda: layer.batch_select_indices(torch.tensor([0]))):
        with pytest.raises(NotImplementedError):
            call()


def test_cpu_model_runs_on_the_package_cpu_path():
    """Without the oracle stand-in a CPU model runs on the package's own CPU library (libkushcpu.so):
    prefill and 12 decode steps give the logits of the oracle-backed run (kushkash/cache.py:72-78: the
    reference's CPU path), within fp32 summation order."""
    model = kk.enable(_tiny("llama"))
    ids = torch.randint(0, 256, (2, 40))
    runs = []
    with torch.no_grad():
        for backend in (None, oracle_backend):
            out = []
            with (backend() if backend else contextlib.nullcontext()):
                cache = kk.KushHFCache(model.config, bits=4)
                logits = model(ids, past_key_values=cache, use_cache=True).logits
                out.append(logits)
                nxt = logits[:, -1:].argmax(-1)
                for _ in range(12):
                    logits = model(nxt, past_key_values=cache, use_cache=True).logits
                    out.append(logits)
                    nxt = logits.argmax(-1)
            runs.append(torch.cat(out, 1))
            if backend is None:
                assert type(cache.kv.ops) is kk.Ops and not cache.kv.ops.gpu     # the package's own CPU path
    assert torch.allclose(runs[0], runs[1], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("kind", ["llama", "qwen2"])
def test_hf_generate(kind, oracle):
    """tests/test_cpu.py:122-142: prefill is exact; int8 decode steps stay within 5 % of the largest
    DynamicCache logit for 40 steps."""
    from transformers import DynamicCache
    model = _tiny(kind)
    ids = torch.randint(0, 256, (2, 75))
    with torch.no_grad():
        ref = model(ids, past_key_values=DynamicCache(config=model.config), use_cache=True)
        kk.enable(model)
        cache = kk.KushHFCache(model.config, bits=8)
        out = model(ids, past_key_values=cache, use_cache=True)
        assert torch.allclose(out.logits, ref.logits, atol=1e-4)
        assert cache.get_seq_length() == 75
        rc, nxt = ref.past_key_values, out.logits[:, -1:].argmax(-1)
        for _ in range(40):
            a = model(nxt, past_key_values=cache, use_cache=True).logits
            model.set_attn_implementation("sdpa")
            r = model(nxt, past_key_values=rc, use_cache=True).logits
            kk.enable(model)
            assert (a - r).abs().max() < 0.05 * r.abs().max()
            nxt = r.argmax(-1)
        assert cache.get_seq_length() == 115


def test_hf_chunked_prefill_and_generate(oracle):
    """tests/test_cpu.py:145-158: a chunk over quantized history matches full attention; model.generate
    runs on a 4-bit cache."""
    model = kk.enable(_tiny("llama"))
    ids = torch.randint(0, 256, (1, 100))
    with torch.no_grad():
        cache = kk.KushHFCache(model.config, bits=8)
        model(ids[:, :60], past_key_values=cache, use_cache=True)
        b = model(ids[:, 60:], past_key_values=cache, use_cache=True).logits
        model.set_attn_implementation("sdpa")
        full = model(ids, use_cache=False).logits[:, 60:]
        assert (b - full).abs().max() < 0.05 * full.abs().max()
        kk.enable(model)
        gen = model.generate(ids, past_key_values=kk.KushHFCache(model.config, bits=4), max_new_tokens=20,
                             do_sample=False)
        assert gen.shape == (1, 120)


def test_reused_cache(oracle):
    """tests/test_cpu.py:212-232: a used cache only continues its own sequence; multi-turn and reset()
    work, and an empty cache accepts a RoPE offset."""
    model = kk.enable(_tiny("llama"))
    p, turn = torch.randint(1, 256, (1, 20)), torch.randint(1, 256, (1, 10))
    g = dict(max_new_tokens=6, do_sample=False)
    with torch.no_grad():
        cache = kk.KushHFCache(model.config, bits=8)
        first = model.generate(p, past_key_values=cache, **g)
        with pytest.raises(RuntimeError, match="holds 25 tokens"):
            model.generate(p, past_key_values=cache, **g)
        assert cache.get_seq_length() == 25
        nxt = model.generate(torch.cat([first, turn], 1), past_key_values=cache, **g)
        assert nxt.shape == (1, 26 + 10 + 6)
        cache.reset()
        assert torch.equal(model.generate(p, past_key_values=cache, **g), first)
        cache.reset()
        model(p, position_ids=torch.arange(5, 25)[None], past_key_values=cache, use_cache=True)
        assert cache.get_seq_length() == 20


def test_generate_needs_gpu_inputs():
    model = _tiny("llama")
    with pytest.raises(ValueError, match="GPU"):
        kk.generate(model, torch.randint(0, 256, (1, 8)), 4)


def test_pick_greedy_and_sampling():
    """generate's token choice (_generate.py:23-30): greedy is argmax; sampling with top_k = 1 is argmax
    too; top_k never picks outside the k largest logits."""
    from kushkash_amd._generate import _pick
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(4, 50, generator=g)
    assert torch.equal(_pick(logits, False, 1.0, 0), logits.argmax(-1))
    torch.manual_seed(1)
    assert torch.equal(_pick(logits, True, 0.7, 1), logits.argmax(-1))
    top3 = logits.topk(3, -1).indices
    for _ in range(20):
        tok = _pick(logits, True, 1.5, 3)
        assert bool((top3 == tok[:, None]).any(-1).all())
