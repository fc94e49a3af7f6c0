"""vLLM plugin registration and ``turboquant_*`` kv-cache-dtype presets
(reference ``vllm_plugin/plugin.py:32-481``).

``register_backend()`` is the ``vllm.general_plugins`` entry point: it puts
``FusedTurboQuantV1Backend`` in vLLM v1's ``AttentionBackendEnum.TURBOQUANT``
slot when vLLM is importable and returns whether it did.

Cache dtypes: the stock presets ``turboquant_3bit_nc`` (K3V3),
``turboquant_k3v4_nc`` and ``turboquant_4bit_nc`` (K4V4) size the slot; the
extended aliases ``turboquant_k{K}v{V}_nc`` (K, V in 2..4) map to the smallest
stock preset whose slot holds them, with the effective widths carried in
``TURBOQUANT_KEY_BITS`` / ``TURBOQUANT_VALUE_BITS`` (the reference's
mechanism, ``plugin.py:380-412``).
"""
from __future__ import annotations

import logging
import os
import re

logger = logging.getLogger(__name__)

# stock preset -> (key bits, value bits) of its slot
TQ_PRESETS = {
    "turboquant_3bit_nc": (3, 3),
    "turboquant_k3v4_nc": (3, 4),
    "turboquant_4bit_nc": (4, 4),
}
_KV_ALIAS = re.compile(r"^turboquant_k([1-4])v([1-4])_nc$")

# additional_config["turboquant"] keys -> environment variables (reference plugin.py:328-339)
TQ_CONFIG_ENV_MAP = {
    "kind": "TURBOQUANT_KIND",
    "boundary_protect": "TURBOQUANT_BOUNDARY_PROTECT",
    "v_rotate": "TURBOQUANT_V_ROTATE",
    "v_lloyd_max": "TURBOQUANT_V_LLOYD_MAX",
    "key_bits": "TURBOQUANT_KEY_BITS",
    "value_bits": "TURBOQUANT_VALUE_BITS",
    "defer_prefill": "TURBOQUANT_DEFER_PREFILL",
}


def host_preset(kv_cache_dtype: str) -> tuple[str, int, int]:
    """(stock preset, effective K bits, effective V bits) of a cache dtype.

    Effective bits: ``TURBOQUANT_KEY_BITS`` / ``_VALUE_BITS`` when set, else
    the alias's own K/V, else the preset's.  Raises ``ValueError`` for an
    unknown dtype or an override wider than the preset's slot.
    """
    m = _KV_ALIAS.match(kv_cache_dtype)
    if m:
        k, v = int(m.group(1)), int(m.group(2))
        preset = ("turboquant_3bit_nc" if k <= 3 and v <= 3 else
                  "turboquant_k3v4_nc" if k <= 3 and v <= 4 else "turboquant_4bit_nc")
    elif kv_cache_dtype in TQ_PRESETS:
        preset = kv_cache_dtype
        k, v = TQ_PRESETS[preset]
    else:
        raise ValueError(f"unknown TurboQuant kv_cache_dtype {kv_cache_dtype!r}")
    pk, pv = TQ_PRESETS[preset]
    k = int(os.environ.get("TURBOQUANT_KEY_BITS", k))
    v = int(os.environ.get("TURBOQUANT_VALUE_BITS", v))
    if not (2 <= k <= 4 and 2 <= v <= 4):
        raise ValueError(f"TurboQuant K/V bits must be 2, 3 or 4 on gfx950; got K={k}, V={v}")
    if k > pk or v > pv:
        raise ValueError(f"K={k}, V={v} exceeds the slot of preset {preset} (K={pk}, V={pv}); "
                         "pick a larger preset such as turboquant_4bit_nc")
    return preset, k, v


def env_flag(name: str, default: bool = False) -> bool:
    raw = os.environ.get(name)
    if raw is None:
        return default
    return raw.strip().lower() in ("1", "true", "yes", "on")


def boundary_protect_mode() -> "str | int":
    """``TURBOQUANT_BOUNDARY_PROTECT`` (reference ``plugin.py:64-118``):
    ``"off"`` (0/off/false/no), ``"fp16"`` (1/fp16/f16/bf16/bfloat16, the
    default: vLLM keeps the first and last attention layers at raw fp16 slots),
    ``"fp8"`` (fp8/f8), or a bit count in {2, 3, 4, 8} (boundary layers stored
    as TurboQuant codes at that width in their fp16-sized slot).  Anything else
    raises ``ValueError``."""
    raw = os.environ.get("TURBOQUANT_BOUNDARY_PROTECT", "1").strip().lower()
    if raw in ("0", "false", "off", "no"):
        return "off"
    if raw in ("1", "fp16", "f16", "bf16", "bfloat16"):
        return "fp16"
    if raw in ("fp8", "f8"):
        return "fp8"
    try:
        bits = int(raw)
    except ValueError as e:
        raise ValueError(f"TURBOQUANT_BOUNDARY_PROTECT={raw!r} not understood. Use 0/off, "
                         "1/fp16, fp8, or a bit count from {2, 3, 4, 8}.") from e
    if bits not in (2, 3, 4, 8):
        raise ValueError(f"TURBOQUANT_BOUNDARY_PROTECT={bits} not supported. Use one of {{2, 3, 4, 8}} "
                         "for a quantized boundary, or 1/fp16 or fp8 for raw / FP8 boundary.")
    return bits


def boundary_protect_enabled() -> bool:
    """Boolean view of ``boundary_protect_mode`` (reference ``plugin.py:120-122``):
    any mode but ``"off"`` keeps boundary layers in fp16-sized slots, which
    widens the shared slot to 2*head_size bf16 elements."""
    return boundary_protect_mode() != "off"


def apply_additional_config(engine_args) -> None:
    """Project ``engine_args.additional_config["turboquant"]`` onto the
    environment variables above (explicit environment values win)."""
    extra = getattr(engine_args, "additional_config", None) or {}
    tq = extra.get("turboquant") if isinstance(extra, dict) else None
    if not isinstance(tq, dict):
        return
    for key, env in TQ_CONFIG_ENV_MAP.items():
        if tq.get(key) is not None:
            val = tq[key]
            os.environ.setdefault(env, ("1" if val else "0") if isinstance(val, bool) else str(val))


def register_backend() -> bool:
    """vLLM entry point: register the v1 backend under ``TURBOQUANT``."""
    try:
        from vllm.v1.attention.backends.registry import AttentionBackendEnum
        from vllm.v1.attention.backends.registry import register_backend as v1_register
    except ImportError:
        logger.debug("vLLM v1 attention registry not importable; TURBOQUANT backend not registered")
        return False
    v1_register(AttentionBackendEnum.TURBOQUANT,
                "fused_turboquant.vllm_plugin.v1_backend.FusedTurboQuantV1Backend")
    return True
