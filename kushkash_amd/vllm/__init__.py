"""vLLM plugin: the kushkash attention backend, bound to vLLM's CUSTOM backend slot, on the gfx950 kernels.

    vllm serve <model> --attention-backend CUSTOM      # KUSHKASH_BITS=4 (default) or 8

vLLM runs ``register`` in every process through its ``vllm.general_plugins`` entry point (declared as
``kushkash_amd = "kushkash_amd.vllm:register"``). kv_cache_dtype stays "auto": the backend declares its
own page size (``KushAttentionBackend.customize_spec``), so vLLM's block manager allocates record-sized
pages and its capacity and concurrency figures count them. Reference: kushkash/vllm/__init__.py:1-57.
"""
from __future__ import annotations

import contextvars
import functools
import inspect

BACKEND = "kushkash_amd.vllm.backend.KushAttentionBackend"

# the request-state indices of the batch being prepared (see patch_hybrid_req_idx)
_BATCH_REQ_IDX: contextvars.ContextVar = contextvars.ContextVar("kushkash_amd_req_idx", default=None)


def register() -> None:
    """Bind vLLM's CUSTOM attention backend to this one; pass req_idx on for hybrid models."""
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend
    register_backend(AttentionBackendEnum.CUSTOM, BACKEND)
    patch_hybrid_req_idx()


def patch_hybrid_req_idx() -> bool:
    """The backend keys each request's exact K tail on req_idx, the request-state index vLLM's model
    runner V2 passes into the attention metadata. Its hybrid (Mamba / linear-attention) model state
    builds that metadata without it; this wraps its ``prepare_attn`` to keep the batch's index mapping
    (``input_batch.idx_mapping_np``) for the duration of the call and its ``build_attn_metadata`` to
    pass it as req_idx when none is given. True when the wrap is (already) in place; False when this
    vLLM has no such model state or its builder takes no req_idx (nothing to do)."""
    try:
        from vllm.v1.worker.gpu.model_states import mamba_hybrid as hybrid
    except Exception:                                  # another vLLM layout or platform: the plugin still loads
        return False
    if getattr(hybrid, "_kushkash_amd_req_idx", False):
        return True
    state = getattr(hybrid, "MambaHybridModelState", None)
    build = getattr(hybrid, "build_attn_metadata", None)
    if state is None or build is None or "req_idx" not in inspect.signature(build).parameters:
        return False
    prepare = state.prepare_attn

    @functools.wraps(prepare)
    def prepare_attn(self, input_batch, *args, **kwargs):
        token = _BATCH_REQ_IDX.set(input_batch.idx_mapping_np)
        try:
            return prepare(self, input_batch, *args, **kwargs)
        finally:
            _BATCH_REQ_IDX.reset(token)

    @functools.wraps(build)
    def build_attn_metadata(*args, **kwargs):
        if kwargs.get("req_idx") is None:
            kwargs["req_idx"] = _BATCH_REQ_IDX.get()
        return build(*args, **kwargs)

    state.prepare_attn = prepare_attn
    hybrid.build_attn_metadata = build_attn_metadata
    hybrid._kushkash_amd_req_idx = True
    return True
