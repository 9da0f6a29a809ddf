"""kushkash_amd: the compressed-KV hot path of kushkash (paged int4 / int8 KV cache with fused
dequant decode attention) as hand-written HIP kernels for AMD Instinct MI355X (gfx950).

Drop-in for the reference's kushkash.KushCache / kushkash._ops.Ops on one GPU, for its Hugging Face
entry points (KushHFCache, enable, generate; transformers is imported on first use) and for its
SGLang plugin (kushkash_amd.sglang; SGLang is imported when the plugin registers)."""
from ._ops import PAGE, Ops, record_bytes
from .cache import KushCache, MemoryStats

__all__ = ["KushCache", "MemoryStats", "PAGE", "Ops", "record_bytes", "KushHFCache", "enable", "generate", "build"]
__version__ = "0.1.0"


def __getattr__(name):
    if name in ("KushHFCache", "enable"):
        from . import hf
        return getattr(hf, name)
    if name == "generate":
        from ._generate import generate
        return generate
    raise AttributeError(name)


def build(verbose: bool = False):
    """Compile the gfx950 HIP library in place (hipcc); returns its path."""
    from .build import build as _build
    return _build(verbose=verbose)
