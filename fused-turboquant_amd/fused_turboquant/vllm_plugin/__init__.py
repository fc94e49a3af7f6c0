"""vLLM plugin: the ``TURBOQUANT`` attention backend on the gfx950 kernels
(reference ``vllm_plugin/__init__.py``).

Usage::

    vllm serve <model> --attention-backend TURBOQUANT --kv-cache-dtype turboquant_3bit_nc

``register_backend`` is the ``vllm.general_plugins`` entry point; it also runs
on import so every vLLM process that touches the package registers the
backend.  Environment variables: ``TURBOQUANT_KEY_BITS`` /
``TURBOQUANT_VALUE_BITS`` (per-K/V bit overrides inside the preset's slot),
``TURBOQUANT_V_ROTATE`` (Hadamard-rotate V before its uniform quantisation),
``TURBOQUANT_BOUNDARY_PROTECT`` (boundary layers: raw fp16 slots by default,
or TurboQuant codes at 2/3/4 bits).
"""
from .plugin import (TQ_PRESETS, apply_additional_config, boundary_protect_enabled, boundary_protect_mode,
                     env_flag, host_preset, register_backend)
from .v1_backend import FusedTurboQuantV1Backend, FusedTurboQuantV1Impl

__all__ = ["register_backend", "host_preset", "TQ_PRESETS", "apply_additional_config",
           "boundary_protect_enabled", "boundary_protect_mode", "env_flag", "FusedTurboQuantV1Backend",
           "FusedTurboQuantV1Impl"]

try:
    register_backend()
except Exception:  # pragma: no cover - depends on the installed vLLM
    import logging
    logging.getLogger(__name__).debug("TURBOQUANT backend auto-registration failed", exc_info=True)
