"""vLLM plugin registration and ``turboquant_*`` kv-cache-dtype presets
(reference ``vllm_plugin/plugin.py:32-481``).

``register_backend()`` is the ``vllm.general_plugins`` entry point: it puts
``FusedTurboQuantV1Backend`` in vLLM v1's ``AttentionBackendEnum.TURBOQUANT``
slot when vLLM is importable and returns whether it did.

Cache dtypes: the stock presets ``turboquant_3bit_nc`` (K3V3),
``turboquant_k3v4_nc`` and ``turboquant_4bit_nc`` (K4V4) size the slot; the
extended aliases ``turboquant_k{K}v{V}_nc`` (K, V in 1..4) map to the smallest
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
    if not (1 <= k <= 4 and 1 <= v <= 4):
        raise ValueError(f"TurboQuant K/V bits must be in 1..4; got K={k}, V={v}")
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


def remap_kv_cache_dtype(value):
    """An extended alias ``turboquant_k{K}v{V}_nc`` -> the smallest stock
    preset whose slot holds it, with ``TURBOQUANT_KEY_BITS`` /
    ``TURBOQUANT_VALUE_BITS`` set to K / V unless already set (reference
    ``_ft_remap_kv_cache_dtype``, ``plugin.py:380-412``).  Anything else is
    returned unchanged."""
    if not isinstance(value, str):
        return value
    m = _KV_ALIAS.match(value)
    if not m:
        return value
    k, v = int(m.group(1)), int(m.group(2))
    host = ("turboquant_3bit_nc" if k <= 3 and v <= 3 else
            "turboquant_k3v4_nc" if k <= 3 and v <= 4 else "turboquant_4bit_nc")
    os.environ.setdefault("TURBOQUANT_KEY_BITS", str(k))
    os.environ.setdefault("TURBOQUANT_VALUE_BITS", str(v))
    logger.info("fused-turboquant: kv_cache_dtype %s -> %s (K=%d, V=%d)", value, host, k, v)
    return host


def _mark(fn):
    fn._fused_tq_patched = True
    return fn


def _patched(fn) -> bool:
    fn = getattr(fn, "__func__", fn)
    return bool(getattr(fn, "_fused_tq_patched", False))


def patch_kv_cache_spec() -> bool:
    """Every attention layer whose kv_cache_dtype is ``turboquant_*`` reports
    a ``TQFullAttentionSpec`` of uint8 elements whose ``tq_slot_size`` is the
    backend's own ``_slot_size_for`` (a power of two), so vLLM's page size and
    ``get_kv_cache_shape`` agree; other layers' specs are left alone (they
    belong to other backends and their own layouts).  Reference
    ``_patch_attention_get_kv_cache_spec``, ``plugin.py:165-259``."""
    try:
        import torch
        from vllm.model_executor.layers.attention import attention as attn_mod  # type: ignore
        from vllm.v1.kv_cache_interface import (  # type: ignore
            FullAttentionSpec, SlidingWindowSpec, TQFullAttentionSpec)
    except ImportError:
        return False
    from .v1_backend import FusedTurboQuantV1Backend
    Attention = attn_mod.Attention
    if _patched(Attention.get_kv_cache_spec):
        return True
    original = Attention.get_kv_cache_spec

    def get_kv_cache_spec(self, *args, **kwargs):
        spec = original(self, *args, **kwargs)
        dt = getattr(self, "kv_cache_dtype", "auto") or "auto"
        if not (isinstance(dt, str) and dt.startswith("turboquant_")):
            return spec
        if not isinstance(spec, (TQFullAttentionSpec, SlidingWindowSpec, FullAttentionSpec)):
            return spec
        return TQFullAttentionSpec(block_size=spec.block_size, num_kv_heads=spec.num_kv_heads,
                                   head_size=spec.head_size,
                                   head_size_v=getattr(spec, "head_size_v", spec.head_size),
                                   dtype=torch.uint8,
                                   tq_slot_size=FusedTurboQuantV1Backend._slot_size_for(self.head_size, dt))

    Attention.get_kv_cache_spec = _mark(get_kv_cache_spec)
    return True


def unify_page_sizes(kv_cache_spec: dict) -> dict:
    """Layers whose page is smaller than the largest by an integer ratio get
    their block_size multiplied by that ratio, so every layer's page has the
    same bytes (the slot sizes here are powers of two, so the ratios are
    integers); any other mismatch raises ``NotImplementedError``.  Reference
    ``_patch_unify_page_size``, ``plugin.py:262-319``."""
    from dataclasses import replace
    sizes = {spec.page_size_bytes for spec in kv_cache_spec.values()}
    if len(sizes) <= 1:
        return kv_cache_spec
    top = max(sizes)
    out = {}
    for name, spec in kv_cache_spec.items():
        ps = spec.page_size_bytes
        if ps == top:
            out[name] = spec
            continue
        if top % ps:
            raise NotImplementedError(f"page sizes are not in an integer ratio (largest {top}, {name}: {ps})")
        out[name] = replace(spec, block_size=spec.block_size * (top // ps))
    return out


def patch_unify_page_size() -> bool:
    """Install ``unify_page_sizes`` as vLLM's ``unify_kv_cache_spec_page_size``."""
    try:
        from vllm.v1.core import kv_cache_utils  # type: ignore
    except ImportError:
        return False
    cur = getattr(kv_cache_utils, "unify_kv_cache_spec_page_size", None)
    if cur is None:
        return False
    if not _patched(cur):
        kv_cache_utils.unify_kv_cache_spec_page_size = _mark(lambda spec: unify_page_sizes(spec))
    return True


def patch_boundary_skip_layers() -> bool:
    """With ``TURBOQUANT_BOUNDARY_PROTECT`` off, vLLM's
    ``TurboQuantConfig.get_boundary_skip_layers`` returns no layers, so every
    layer takes the configured ``turboquant_*`` dtype; otherwise vLLM's
    default boundary layers stay.  Reference
    ``_patch_disable_boundary_protection``, ``plugin.py:125-162``."""
    if boundary_protect_enabled():
        return False
    try:
        from vllm.model_executor.layers.quantization.turboquant.config import TurboQuantConfig  # type: ignore
    except ImportError:
        return False
    cur = TurboQuantConfig.__dict__.get("get_boundary_skip_layers")
    if cur is not None and _patched(cur):
        return True

    def get_boundary_skip_layers(num_layers, n=2):
        return []
    TurboQuantConfig.get_boundary_skip_layers = staticmethod(_mark(get_boundary_skip_layers))
    return True


def patch_engine_args() -> bool:
    """``EngineArgs.__post_init__`` first rewrites an extended
    ``turboquant_k{K}v{V}_nc`` cache dtype to its host preset (plus the K / V
    bit variables) and projects ``additional_config["turboquant"]`` onto the
    environment, then runs vLLM's own ``__post_init__`` -- the alias never
    reaches vLLM's Literal check of the cache dtype.  Reference
    ``_patch_extend_tq_presets``, ``plugin.py:415-481`` (its flash-attn
    version forwarding has no counterpart: prefill here runs through SDPA)."""
    try:
        from vllm.engine.arg_utils import EngineArgs  # type: ignore
    except ImportError:
        return False
    if _patched(EngineArgs.__post_init__):
        return True
    original = EngineArgs.__post_init__

    def __post_init__(self):
        for attr in ("kv_cache_dtype", "cache_dtype"):
            cur = getattr(self, attr, None)
            if isinstance(cur, str):
                new = remap_kv_cache_dtype(cur)
                if new is not cur:
                    setattr(self, attr, new)
        apply_additional_config(self)
        original(self)

    __post_init__.__wrapped__ = original
    EngineArgs.__post_init__ = _mark(__post_init__)
    return True


def patch_cache_dtype_validation() -> bool:
    """Kept for the reference's call sequence (``plugin.py:484-491``): vLLM
    validates the cache dtype as a Literal that cannot be widened at run time,
    so the alias is rewritten before validation (``patch_engine_args``) and
    nothing is patched here."""
    return False


def register_backend() -> bool:
    """vLLM entry point: register the v1 backend under ``TURBOQUANT`` and
    install the patches the reference's ``register_backend`` installs
    (``plugin.py:32-61``): kv-cache spec, page-size unification, boundary
    skip layers, extended presets, cache-dtype validation.  Each patch is
    idempotent and a no-op where its vLLM module is missing.  Returns whether
    the backend was registered."""
    try:
        from vllm.v1.attention.backends.registry import AttentionBackendEnum
        from vllm.v1.attention.backends.registry import register_backend as v1_register
    except ImportError:
        logger.debug("vLLM v1 attention registry not importable; TURBOQUANT backend not registered")
        return False
    v1_register(AttentionBackendEnum.TURBOQUANT,
                "fused_turboquant.vllm_plugin.v1_backend.FusedTurboQuantV1Backend")
    patch_kv_cache_spec()
    patch_unify_page_size()
    patch_boundary_skip_layers()
    patch_engine_args()
    patch_cache_dtype_validation()
    return True
