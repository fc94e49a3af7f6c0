"""HuggingFace integration (reference ``src/fused_turboquant/hf/__init__.py``)."""
from .fused_cache import (  # noqa: F401
    CompressedKVCache,
    FusedTurboQuantRunner,
    check_model_compatibility,
    make_fused_attention_forward,
    patch_model,
    unpatch_model,
)
from .chunked_prefill import chunked_generate, chunked_prefill  # noqa: F401

__all__ = ["CompressedKVCache", "FusedTurboQuantRunner", "check_model_compatibility",
           "make_fused_attention_forward", "patch_model", "unpatch_model", "chunked_prefill", "chunked_generate"]
