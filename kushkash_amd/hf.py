"""Hugging Face transformers (>= 5.0) entry point: a transformers ``Cache`` backed by a KushCache and
the "kushkash" attention function that writes to it and attends over it with the HIP kernels.
Contract: kushkash/hf.py:1-220 (same public names, arguments and error behaviour).

    import kushkash_amd as kk
    model = kk.enable(model)                                  # validate, register, select "kushkash"
    out = model.generate(**inputs, past_key_values=kk.KushHFCache(model.config, bits=4), max_new_tokens=256)

Per layer, transformers calls ``Cache.update`` and then the attention function with the same new
K/V chunk. ``KushHFCache.update`` stores nothing: it creates the KushCache on first use and leaves
itself in a thread-local slot, which the attention function takes (the attention interface passes
no cache). The attention function then, by the chunk's length T and the cached length n:
  T = 1          append the token and decode over the cache, in one launch (KushCache.append_attend);
  T > 1, n = 0   exact causal attention over the prompt, then the ragged write of the prompt;
  T > 1, n > 0   attention over the dequantized history, one page block at a time, plus the chunk
                 (causal), merged by log-sum-exp (KushCache.attend_chunk); then the write.
"""
from __future__ import annotations

import threading

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel
from transformers import AttentionInterface, AttentionMaskInterface
from transformers.cache_utils import Cache, CacheLayerMixin

from ._ops import attn_lse
from .cache import KushCache

NAME = "kushkash"
_handoff = threading.local()        # .cache: the KushHFCache whose update() ran last on this thread


def _text_config(config):
    return config.get_text_config() if hasattr(config, "get_text_config") else config


class _KushLayer(CacheLayerMixin):
    """One layer's view of the shared KushCache (hf.py:34-80). It holds no tensors: lengths come
    from the KushCache, and the operations a quantized page cache cannot do raise."""
    is_sliding = False
    is_croppable = False

    def __init__(self, owner: "KushHFCache", layer: int):
        super().__init__()
        self.owner, self.layer = owner, layer

    def lazy_initialization(self, key_states, value_states):
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        return key_states, value_states

    def get_seq_length(self) -> int:
        kv = self.owner.kv
        return 0 if kv is None else kv.length(self.layer)

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        # sizes only: kush_mask never builds a mask (causal over everything cached plus the chunk)
        return self.get_seq_length() + query_length, 0

    def get_max_length(self) -> int:
        return -1                                   # pages are mapped on demand

    def reset(self) -> None:
        if self.layer == 0 and self.owner.kv is not None:
            self.owner.kv.reset()

    def reorder_cache(self, beam_idx):
        raise NotImplementedError("kushkash: beam search is not supported")

    def crop(self, max_length):
        raise NotImplementedError("kushkash: cropping (assisted / speculative decoding) is not supported")

    def batch_repeat_interleave(self, repeats):
        raise NotImplementedError("kushkash: batch expansion is not supported; pass num_return_sequences=1")

    def batch_select_indices(self, indices):
        raise NotImplementedError("kushkash: batch selection is not supported")

    def offload(self):
        pass

    def prefetch(self):
        pass


class KushHFCache(Cache):
    """Drop-in for transformers' DynamicCache (hf.py:83-119).

    Args:
        config: the model config (the text config of a multimodal model is used).
        bits: 4 (default) or 8.
        max_length: optional per-sequence capacity hint (pages are mapped on demand otherwise).
        rotate: Hadamard rotation inside the cache (None: KUSHKASH_ROTATE; auto = on for 4-bit).
        rotate_in_kernels: fold that rotation into the write and decode kernels (KushCache's option of
            the same name; no reference counterpart).
    The KushCache itself is created by the first update(), on the device and in the dtype of the
    model's K/V (a GPU device: the kernels run on the GPU only).
    """

    def __init__(self, config, bits: int = 4, max_length: int | None = None, rotate: bool | None = None,
                 rotate_in_kernels: bool = False):
        cfg = _text_config(config)
        self.num_layers = cfg.num_hidden_layers
        self.num_q_heads = cfg.num_attention_heads
        self.head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self.bits, self.max_length, self.rotate, self.rotate_in_kernels = bits, max_length, rotate, rotate_in_kernels
        self.kv: KushCache | None = None
        super().__init__(layers=[_KushLayer(self, i) for i in range(self.num_layers)])

    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        """Called by transformers right before the attention function of layer `layer_idx`; the chunk
        is written by that function, so it is returned unchanged."""
        if self.kv is None:
            B, H, _, D = key_states.shape
            self.kv = KushCache(self.num_layers, H, self.num_q_heads, D, batch_size=B, bits=self.bits,
                                device=key_states.device, dtype=key_states.dtype, max_length=self.max_length,
                                rotate=self.rotate, rotate_in_kernels=self.rotate_in_kernels)
        self.layers[layer_idx].is_initialized = True
        _handoff.cache = self
        return key_states, value_states

    def memory(self):
        """MemoryStats of the KushCache (None before the first forward)."""
        return None if self.kv is None else self.kv.memory()


def prompt_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal attention of a prompt over itself (nothing cached yet): q [B, Hq, T, D], k, v
    [B, Hkv, T, D] -> [B, Hq, T, D] in q's dtype (hf.py:122-129). fp32 inputs use the fp32 product
    path (attn_lse). fp16 / bf16 take torch's fused SDPA, restricted to its flash and
    memory-efficient kernels, with K/V expanded to the q heads; where neither applies the fp32
    path runs instead, so torch's half-precision math fallback (batched products over transposed
    views) is never used."""
    if q.dtype != torch.float32:
        g = q.shape[1] // k.shape[1]
        ke, ve = (k.repeat_interleave(g, 1), v.repeat_interleave(g, 1)) if g > 1 else (k, v)
        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                return F.scaled_dot_product_attention(q, ke, ve, is_causal=True, scale=scale)
        except RuntimeError:
            pass
    return attn_lse(q, k, v, True, scale)[0].to(q.dtype)


def _check_start(kv: KushCache, position_ids) -> None:
    """A multi-token chunk must continue the sequence the cache holds (hf.py:132-147): generate() on a
    cache that already holds another sequence would attend to it silently. Checked on layer 0 of a
    multi-token forward (one host read), never on decode steps; skipped on an empty cache and
    without 2-D position ids."""
    held = kv.length(0)
    if held == 0 or position_ids is None or position_ids.dim() != 2:
        return
    start = int(position_ids[0, 0])
    if start != held:
        raise RuntimeError(f"kushkash: this KushHFCache holds {held} tokens, but the new input starts at position "
                           f"{start}, not {held}. A cache only continues the sequence it holds (for another turn, "
                           f"pass the earlier ids plus the new ones). Use a new KushHFCache, or cache.reset(), for "
                           f"another prompt.")


def kush_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """The "kushkash" attention function (hf.py:150-177). query [B, Hq, T, D]; key, value: the new
    chunk [B, Hkv, T, D]. Returns ([B, T, Hq, D], None)."""
    owner: KushHFCache | None = getattr(_handoff, "cache", None)
    _handoff.cache = None                           # one update() per attention call
    if owner is None or owner.kv is None:
        raise RuntimeError("kushkash attention needs past_key_values=KushHFCache(...) (and use_cache=True)")
    kv, layer = owner.kv, module.layer_idx
    if scaling is not None:
        kv.scale = float(scaling)
    T = query.shape[2]
    if T == 1:
        return kv.append_attend(layer, query[:, :, 0], key, value).unsqueeze(1), None
    if layer == 0:
        _check_start(kv, kwargs.get("position_ids"))
    if kv.length(layer) == 0:
        out = prompt_attention(query, key, value, kv.scale)
    else:
        out = kv.attend_chunk(layer, query, key, value)
    kv.write(layer, key, value)
    return out.transpose(1, 2).contiguous(), None


def kush_mask(batch_size, q_length, kv_length, *args, attention_mask=None, **kwargs):
    """The "kushkash" mask function (hf.py:180-186): no mask is built, the kernels are causal by
    construction. A padded batch is refused on multi-token calls; decode steps are not checked
    (that would read the mask back every token)."""
    if (attention_mask is not None and q_length > 1 and attention_mask.dim() == 2
            and not bool(attention_mask.all())):
        raise NotImplementedError("kushkash: padded batches are not supported; batch equal-length prompts")
    return None


def _window_binds(cfg) -> bool:
    """Whether the config's attention window can exclude tokens (hf.py:189-206): layer_types decide
    when present (a window applies only to "sliding_attention" layers); without them, the legacy
    use_sliding_window flag, or a sliding_window below max_position_embeddings (a window with no
    maximum to compare against counts as binding)."""
    types = getattr(cfg, "layer_types", None)
    if types:
        return any(t != "full_attention" for t in types)
    if getattr(cfg, "use_sliding_window", False):
        return True
    window = getattr(cfg, "sliding_window", None)
    if not window:
        return False
    limit = getattr(cfg, "max_position_embeddings", None)
    return limit is None or window < limit


def _check_config(config) -> None:
    """Refuse the attention variants the kernels do not compute (hf.py:209-216)."""
    cfg = _text_config(config)
    if _window_binds(cfg):
        raise NotImplementedError("kushkash: sliding-window / hybrid attention layers are not supported")
    if getattr(cfg, "attn_logit_softcapping", None):
        raise NotImplementedError("kushkash: attention logit softcapping is not supported")
    if getattr(cfg, "kv_lora_rank", None):
        raise NotImplementedError("kushkash: MLA (latent KV) models are not supported")


def register() -> None:
    AttentionInterface.register(NAME, kush_attention)
    AttentionMaskInterface.register(NAME, kush_mask)


def enable(model):
    """Validate the model's config, register the "kushkash" attention and select it; returns the model."""
    _check_config(model.config)
    register()
    model.set_attn_implementation(NAME)
    return model
