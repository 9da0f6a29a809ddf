"""Hugging Face transformers (>= 5.0) entry point: KushHFCache, a transformers Cache over a KushCache,
and the "kushkash" attention function that writes each new K / V chunk into it and attends over it
with the gfx950 kernels. Public names, arguments and error types: the reference's hf.py (hf.py:1-220).

    import kushkash_amd as kk
    model = kk.enable(model)                         # check the config, register and select "kushkash"
    out = model.generate(**inputs, past_key_values=kk.KushHFCache(model.config, bits=4), max_new_tokens=256)

How a layer's call flows. transformers calls Cache.update(k, v, layer) and then the attention function
with the same k and v tensors. KushHFCache.update stores nothing; it attaches a route -- (cache,
layer) -- to the key tensor, and the attention function reads the route off the key it receives. No
state outlives the call: a forward without a KushHFCache carries no route and is refused. The
attention function then picks by the chunk length T and the tokens n already cached:
    T = 1          append the token and decode, one kernel launch (KushCache.append_attend);
    T > 1, n = 0   causal attention over the prompt itself, then the chunk write;
    T > 1, n > 0   attention over the history (unpacked a block at a time by the unpack kernel) and
                   the chunk (causal), merged by log-sum-exp (KushCache.attend_chunk); then the write.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel
from transformers import AttentionInterface, AttentionMaskInterface
from transformers.cache_utils import Cache, CacheLayerMixin

from ._attention import self_attention_blocks
from .cache import KushCache

NAME = "kushkash"
_ROUTE = "_kushkash_route"          # attribute of the key tensor that update() hands to the attention


def _text_config(config):
    return config.get_text_config() if hasattr(config, "get_text_config") else config


def _refuse(what: str):
    raise NotImplementedError(f"kushkash: {what} is not supported by a quantized page cache")


class _PagedLayer(CacheLayerMixin):
    """One layer's face of the shared KushCache for transformers (hf.py:34-80): it holds no tensors,
    reports the cached length, and refuses what a quantized page cache cannot do."""
    is_sliding = False
    is_croppable = False

    def __init__(self, owner: "KushHFCache", index: int):
        super().__init__()
        self.owner, self.index = owner, index

    def lazy_initialization(self, key_states, value_states):
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        return key_states, value_states

    def get_seq_length(self) -> int:
        return self.owner.tokens(self.index)

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.get_seq_length() + query_length, 0     # sizes only: no mask is ever built

    def get_max_length(self) -> int:
        return -1                                           # the pool grows on demand

    def reset(self) -> None:
        if self.index == 0 and self.owner.kv is not None:   # one reset for the whole cache
            self.owner.kv.reset()

    def offload(self):
        pass

    def prefetch(self):
        pass

    def reorder_cache(self, beam_idx):
        _refuse("beam search")

    def crop(self, max_length):
        _refuse("cropping (assisted or speculative decoding)")

    def batch_repeat_interleave(self, repeats):
        _refuse("batch expansion (use num_return_sequences=1)")

    def batch_select_indices(self, indices):
        _refuse("batch selection")


class KushHFCache(Cache):
    """A transformers Cache to pass as past_key_values in place of DynamicCache (hf.py:83-119).

    Args:
        config: the model config (for a multimodal model, its text config is used).
        bits: 4 (default) or 8.
        max_length: per-sequence capacity to reserve (the pool grows on demand otherwise).
        rotate: Hadamard rotation inside the cache (None: KUSHKASH_ROTATE; auto = on for 4-bit).
        rotate_in_kernels: let the kernels do that rotation (KushCache's option; no reference counterpart).
    The KushCache is created by the first update(), with the batch size, device and dtype of the
    model's keys (a GPU device: the kernels run on the GPU only).
    """

    def __init__(self, config, bits: int = 4, max_length: int | None = None, rotate: bool | None = None,
                 rotate_in_kernels: bool = False):
        cfg = _text_config(config)
        self.num_layers = cfg.num_hidden_layers
        self.num_q_heads = cfg.num_attention_heads
        self.head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
        self.bits, self.max_length, self.rotate, self.rotate_in_kernels = bits, max_length, rotate, rotate_in_kernels
        self.kv: KushCache | None = None
        super().__init__(layers=[_PagedLayer(self, i) for i in range(self.num_layers)])

    def tokens(self, layer: int) -> int:
        return 0 if self.kv is None else self.kv.length(layer)

    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        """Called right before layer `layer_idx`'s attention: creates the KushCache on first use and
        routes the chunk to the attention function, which writes it; returns k, v unchanged."""
        if self.kv is None:
            B, H, _, D = key_states.shape
            self.kv = KushCache(self.num_layers, H, self.num_q_heads, D, batch_size=B, bits=self.bits,
                                device=key_states.device, dtype=key_states.dtype, max_length=self.max_length,
                                rotate=self.rotate, rotate_in_kernels=self.rotate_in_kernels)
        self.layers[layer_idx].is_initialized = True
        setattr(key_states, _ROUTE, (self, layer_idx))
        return key_states, value_states

    def memory(self):
        """MemoryStats of the KushCache, or None before the first forward."""
        return None if self.kv is None else self.kv.memory()


def prompt_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                     block_bytes: int = 1 << 28) -> torch.Tensor:
    """Causal attention of a prompt over itself when nothing is cached yet: q [B, Hq, T, D], k, v
    [B, Hkv, T, D] -> [B, Hq, T, D] in q's dtype (hf.py:122-129). Half-precision inputs go to torch's
    fused attention, limited to its flash kernel (K / V expanded to the q heads); everything else, and
    any input the flash kernel refuses, to fp32 products over blocks of keys whose memory stays within
    block_bytes. torch's memory-efficient kernel is not allowed: on ROCm its dense and varlen forms are
    the same kernel family, and its varlen form with a bottom-right causal mask has taken an
    illegal-address fault on this device. torch's half-precision math path (batched products over
    transposed views) is never taken either."""
    if q.dtype in (torch.float16, torch.bfloat16):
        g = q.shape[1] // k.shape[1]
        ke = k.repeat_interleave(g, 1) if g > 1 else k
        ve = v.repeat_interleave(g, 1) if g > 1 else v
        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                return F.scaled_dot_product_attention(q, ke, ve, is_causal=True, scale=scale)
        except RuntimeError:
            pass
    return self_attention_blocks(q, k, v, scale, block_bytes)[0].to(q.dtype)


def _continues(kv: KushCache, position_ids) -> None:
    """A multi-token chunk on a non-empty cache must start at the cache's length (hf.py:132-147):
    otherwise the cache holds another sequence (a KushHFCache reused for a new prompt) and attending
    to it would be silently wrong. One host read, on layer 0 of multi-token forwards only; an empty
    cache (a RoPE offset is fine there) and non-2-D position ids are not checked."""
    held = kv.length(0)
    if held and position_ids is not None and position_ids.dim() == 2:
        first = int(position_ids[0, 0])
        if first != held:
            raise RuntimeError(f"kushkash: this KushHFCache holds {held} tokens, so new input must start at position "
                               f"{held}, but it starts at {first}. Pass the earlier tokens plus the new ones to "
                               f"continue the conversation, or start another prompt with a new KushHFCache (or "
                               f"cache.reset()).")


def kush_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """The "kushkash" attention function (hf.py:150-177): query [B, Hq, T, D]; key, value the new chunk
    [B, Hkv, T, D]; returns ([B, T, Hq, D], None)."""
    route = getattr(key, _ROUTE, None)
    if route is None or route[0].kv is None:
        raise RuntimeError("kushkash attention runs on a KushHFCache: pass past_key_values=KushHFCache(...) "
                           "and use_cache=True")
    delattr(key, _ROUTE)
    kv, layer = route[0].kv, route[1]
    if scaling is not None:
        kv.scale = float(scaling)
    T = query.shape[2]
    if T == 1:
        return kv.append_attend(layer, query[:, :, 0], key, value).unsqueeze(1), None
    if layer == 0:
        _continues(kv, kwargs.get("position_ids"))
    if kv.length(layer):
        out = kv.attend_chunk(layer, query, key, value)
    else:
        out = prompt_attention(query, key, value, kv.scale)
    kv.write(layer, key, value)
    return out.transpose(1, 2).contiguous(), None


def kush_mask(batch_size, q_length, kv_length, *args, attention_mask=None, **kwargs):
    """The "kushkash" mask function (hf.py:180-186): no mask is built (the kernels are causal by
    construction). A padded batch is refused where it shows, on multi-token calls; decode steps are
    not checked (that would read the mask back on every token)."""
    padded = (attention_mask is not None and q_length > 1 and attention_mask.dim() == 2
              and not bool(attention_mask.all()))
    if padded:
        raise NotImplementedError("kushkash: padded batches are not supported; batch prompts of equal length")
    return None


def _window_can_bind(cfg) -> bool:
    """Whether an attention window of the config can hide tokens (hf.py:189-206). Per-layer types, when
    given, decide alone (a window applies to "sliding_attention" layers only). Without them: the
    use_sliding_window flag, or a positive sliding_window shorter than max_position_embeddings (with
    no maximum to compare against, a window is taken to bind)."""
    kinds = getattr(cfg, "layer_types", None)
    if kinds:
        return any(kind != "full_attention" for kind in kinds)
    if getattr(cfg, "use_sliding_window", False):
        return True
    window = getattr(cfg, "sliding_window", None) or 0
    limit = getattr(cfg, "max_position_embeddings", None)
    return window > 0 and (limit is None or window < limit)


# (test on the text config, what is refused): attention these kernels do not compute (hf.py:209-216)
_UNSUPPORTED = (
    (_window_can_bind, "sliding-window / hybrid attention layers"),
    (lambda cfg: bool(getattr(cfg, "attn_logit_softcapping", None)), "attention logit softcapping"),
    (lambda cfg: bool(getattr(cfg, "kv_lora_rank", None)), "MLA (latent KV) attention"),
)


def _check_config(config) -> None:
    cfg = _text_config(config)
    for test, what in _UNSUPPORTED:
        if test(cfg):
            _refuse(what)


def register() -> None:
    AttentionInterface.register(NAME, kush_attention)
    AttentionMaskInterface.register(NAME, kush_mask)


def enable(model):
    """Check the model's config, register the "kushkash" attention and mask functions and select them;
    returns the model."""
    _check_config(model.config)
    register()
    model.set_attn_implementation(NAME)
    return model
