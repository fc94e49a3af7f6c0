"""HuggingFace integration: compressed KV cache + decode attention on gfx950.

Mirrors the reference's ``hf/fused_cache.py`` surface (``patch_model``,
``unpatch_model``, ``CompressedKVCache``, ``check_model_compatibility``,
``FusedTurboQuantRunner``; reference ``hf/fused_cache.py:140-1320``) for the
RHT quantizer.  What differs is underneath:

* K and V of a patched layer live in this library's paged format
  (``fused_turboquant.paged``: pages of 16 tokens per kv head, codes + fp16
  norms), grown by doubling a preallocated buffer -- not re-concatenated on
  every step (the reference appends with ``torch.cat``, ``:195-222``).
* A single-token decode step runs the fused paged decode-attention kernel:
  softmax(q . K^T * scale) . V over the decoded cache without materialising
  K, V or the scores (the reference scores with a fused kernel, then runs
  softmax and a matmul over the bulk-decoded V, ``:576-624``).
* Prefill (q_len > 1 on an empty cache) attends over the full-precision K/V
  with SDPA, as the reference does (``:626-670``), and stores the compressed
  K/V.  A multi-token step on a non-empty cache attends over the decoded past
  plus the new tokens.

Per-sequence lengths: tokens masked out by the attention mask at prefill (left
padding) are not stored, so each sequence's cache holds only its real tokens;
decode steps append one token per sequence.

Layers whose V is kept uncompressed (``compress_v=False`` / ``"boundary"`` /
a callable) keep K in pages and V in full precision; their decode step
dequantises K with the decode kernel and attends with torch ops.
"""
from __future__ import annotations

import logging
import math
from typing import Optional

import torch
import torch.nn.functional as F
from transformers import DynamicCache

from .. import paged as P
from ..core.quantizer import CompressedTensor, TurboQuantMSE

logger = logging.getLogger(__name__)

KNOWN_COMPATIBLE = {
    "LlamaForCausalLM", "MistralForCausalLM", "Qwen2ForCausalLM", "Qwen3ForCausalLM",
    "Gemma2ForCausalLM", "Phi3ForCausalLM",
}

_SKIP_NAME_KEYWORDS = ("encoder_attn", "crossattention", "cross_attn", "visual", "vision_model",
                       "vision_tower", "image_encoder", "vit", "img_attn")
_PAGE = 16


# --------------------------------------------------------------------------
# per-layer paged storage
# --------------------------------------------------------------------------

class _LayerPages:
    """Pages of one layer: sequence b owns blocks [b * cap, (b + 1) * cap), so
    its block-table row is b * cap + arange(cap) and token i of it sits in slot
    b * cap * 16 + i."""

    def __init__(self, batch: int, hkv: int, d: int, k_tq: TurboQuantMSE, v_tq: TurboQuantMSE,
                 device):
        self.B, self.hkv, self.d = batch, hkv, d
        self.k_tq, self.v_tq = k_tq, v_tq
        self.cap = 0
        self.kv_cache: Optional[torch.Tensor] = None
        self.block_table: Optional[torch.Tensor] = None
        self.lens = [0] * batch
        self.lens_dev = torch.zeros(batch, dtype=torch.int32, device=device)
        self.device = device

    def _ensure(self, need_tokens: int) -> None:
        need = (need_tokens + _PAGE - 1) // _PAGE
        if need <= self.cap:
            return
        new_cap = max(need, 2 * self.cap, 4)
        shape = P.cache_shape(self.B * new_cap, _PAGE, self.hkv, self.d, self.k_tq.bits, self.v_tq.bits)
        fresh = torch.zeros(shape, dtype=torch.uint8, device=self.device)
        if self.kv_cache is not None:
            fresh.view(self.B, new_cap, *shape[1:])[:, :self.cap] = self.kv_cache.view(self.B, self.cap, *shape[1:])
        self.kv_cache = fresh
        self.cap = new_cap
        self.block_table = (torch.arange(self.B, device=self.device, dtype=torch.int32).view(-1, 1) * new_cap
                            + torch.arange(new_cap, device=self.device, dtype=torch.int32).view(1, -1))

    def append(self, key: torch.Tensor, value: torch.Tensor, keep: Optional[torch.Tensor]) -> None:
        """key/value [B, Hkv, q, d]; keep [B, q] bool (None = every token)."""
        B, hkv, q, d = key.shape
        if keep is None:
            self._ensure(max(self.lens) + q)
            # slots computed on the device: no host round trip per decode step
            base = torch.arange(B, device=self.device, dtype=torch.int64) * (self.cap * _PAGE)
            slot_t = (base.view(-1, 1) + self.lens_dev.view(-1, 1).to(torch.int64)
                      + torch.arange(q, device=self.device, dtype=torch.int64).view(1, -1)).reshape(-1)
            self.lens = [L + q for L in self.lens]
            new_lens = None
        else:
            keep_l = keep.tolist()
            counts = [sum(1 for k in row if k) for row in keep_l]
            self._ensure(max(L + c for L, c in zip(self.lens, counts)))
            slots = []
            for b in range(B):
                pos, base = self.lens[b], b * self.cap * _PAGE
                for i in range(q):
                    if keep_l[b][i]:
                        slots.append(base + pos)
                        pos += 1
                    else:
                        slots.append(-1)  # masked-out token: skipped by the store kernel
            slot_t = torch.tensor(slots, dtype=torch.int64, device=self.device)
            self.lens = [L + c for L, c in zip(self.lens, counts)]
            new_lens = torch.tensor(self.lens, dtype=torch.int32)
        k = key.permute(0, 2, 1, 3).reshape(B * q, hkv, d)
        v = value.permute(0, 2, 1, 3).reshape(B * q, hkv, d)
        P.paged_store(k, v, self.kv_cache, slot_t, self.k_tq, self.v_tq)
        if new_lens is None:
            self.lens_dev.add_(q)
        else:
            self.lens_dev.copy_(new_lens)

    def flat(self):
        """(K packed, K norms, V packed, V norms) as [B, Hkv, max_len, *]."""
        L = max(self.lens) if self.lens else 0
        pages = (L + _PAGE - 1) // _PAGE
        blocks = self.block_table[:, :pages].reshape(-1)
        kp, kn, vp, vn = P.paged_read(self.kv_cache, blocks, self.d, self.k_tq.bits, self.v_tq.bits)

        def fold(t):  # [B*pages, Hkv, 16, ...] -> [B, Hkv, pages*16, ...][:, :, :L]
            t = t.view(self.B, pages, self.hkv, _PAGE, *t.shape[3:]).transpose(1, 2)
            return t.reshape(self.B, self.hkv, pages * _PAGE, *t.shape[4:])[:, :, :L]
        return fold(kp), fold(kn), fold(vp), fold(vn)


class CompressedKVCache(DynamicCache):
    """KV cache holding TurboQuant-compressed K (and V) per patched layer.

    Reference surface: ``hf/fused_cache.py:140-360`` (per-layer K / V
    quantizers, ``store_compressed_*``, ``get_compressed_*``,
    ``decode_values``, ``reset``).  A dummy one-element slice goes through
    ``DynamicCache.update`` so the base class keeps counting the sequence
    length, as the reference does.
    """

    def __init__(self, quantizer: TurboQuantMSE, compress_v: bool = True):
        super().__init__()
        self.tq = quantizer
        self._layer_tq: dict[int, TurboQuantMSE] = {}
        self._layer_tq_v: dict[int, TurboQuantMSE] = {}
        self.compress_v = compress_v
        self._pages: dict[int, _LayerPages] = {}

    # -- quantizer registry (reference :167-190) ---------------------------
    def set_layer_quantizer(self, layer_idx: int, tq: TurboQuantMSE) -> None:
        self._layer_tq[layer_idx] = tq

    def set_layer_quantizer_v(self, layer_idx: int, tq: TurboQuantMSE) -> None:
        self._layer_tq_v[layer_idx] = tq

    def get_layer_quantizer(self, layer_idx: int) -> TurboQuantMSE:
        return self._layer_tq.get(layer_idx, self.tq)

    def get_layer_quantizer_v(self, layer_idx: int) -> TurboQuantMSE:
        if layer_idx in self._layer_tq_v:
            return self._layer_tq_v[layer_idx]
        return self._layer_tq.get(layer_idx, self.tq)

    # -- storage -------------------------------------------------------------
    def _layer(self, layer_idx: int, like: torch.Tensor) -> _LayerPages:
        lp = self._pages.get(layer_idx)
        if lp is None:
            B, hkv, _, d = like.shape
            lp = _LayerPages(B, hkv, d, self.get_layer_quantizer(layer_idx),
                             self.get_layer_quantizer_v(layer_idx), like.device)
            self._pages[layer_idx] = lp
        return lp

    def store_compressed_kv(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
                            keep: Optional[torch.Tensor] = None) -> None:
        """Encode and append key/value states [B, Hkv, q, d] (one store kernel
        for K and V; ``keep`` [B, q] drops masked-out tokens)."""
        if key_states.shape != value_states.shape:
            raise ValueError("key and value states must have the same shape")
        self._layer(layer_idx, key_states).append(key_states, value_states, keep)

    def store_compressed_key(self, key_states: torch.Tensor, layer_idx: int) -> None:
        """K only: V slots of the pages are filled with zeros (their decode is unused)."""
        self.store_compressed_kv(key_states, torch.zeros_like(key_states), layer_idx)

    def store_compressed_value(self, value_states: torch.Tensor, layer_idx: int) -> None:
        raise NotImplementedError(
            "values are stored together with keys in this cache's pages; use store_compressed_kv")

    def seq_lens(self, layer_idx: int) -> list:
        lp = self._pages.get(layer_idx)
        return list(lp.lens) if lp is not None else []

    def _entry(self, layer_idx: int, which: str) -> Optional[dict]:
        lp = self._pages.get(layer_idx)
        if lp is None:
            return None
        kp, kn, vp, vn = lp.flat()
        if which == "k":
            return {"packed_indices": kp, "norms": kn}
        return {"packed_indices": vp, "norms": vn}

    def get_compressed_key(self, layer_idx: int) -> Optional[dict]:
        """{"packed_indices": [B, Hkv, S, d*bits/8] u8, "norms": [B, Hkv, S] f16};
        positions past a sequence's own length are padding."""
        return self._entry(layer_idx, "k")

    def get_compressed_value(self, layer_idx: int) -> Optional[dict]:
        return self._entry(layer_idx, "v")

    def decode_keys(self, layer_idx: int) -> torch.Tensor:
        tq = self.get_layer_quantizer(layer_idx)
        e = self._entry(layer_idx, "k")
        return tq.decode(CompressedTensor(e["packed_indices"], e["norms"], tq.head_dim, tq.bits))

    def decode_values(self, layer_idx: int) -> torch.Tensor:
        """All cached values of a layer, [B, Hkv, S, d] float32 (reference :333-348)."""
        tq = self.get_layer_quantizer_v(layer_idx)
        e = self._entry(layer_idx, "v")
        return tq.decode(CompressedTensor(e["packed_indices"], e["norms"], tq.head_dim, tq.bits))

    def decode_attention(self, query: torch.Tensor, layer_idx: int, scale: float) -> torch.Tensor:
        """query [B, Hq, d] -> [B, Hq, d] (query dtype), fused over the pages."""
        lp = self._pages[layer_idx]
        return P.paged_decode_attention(query, lp.kv_cache, lp.block_table, lp.lens_dev, lp.k_tq, lp.v_tq,
                                        scale=scale, max_seq_len=max(lp.lens))

    def reset(self):
        """Drop every layer so the object can serve a new prompt (reference :350-360)."""
        self._pages.clear()
        self.layers.clear()


# --------------------------------------------------------------------------
# attention forward
# --------------------------------------------------------------------------

def _rotate_half(x):
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def _apply_rotary_pos_emb(q, k, cos, sin):
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    return (q * cos) + (_rotate_half(q) * sin), (k * cos) + (_rotate_half(k) * sin)


def _repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    if n_rep == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def _keep_from_mask(attention_mask, q_len: int) -> Optional[torch.Tensor]:
    """[B, q] bool of the new tokens a sequence attends to from its last
    query row (False = padding), or None when nothing is masked."""
    if attention_mask is None or attention_mask.dim() != 4:
        return None
    last = attention_mask[:, 0, -1, -q_len:]
    keep = last if last.dtype == torch.bool else (last == 0)
    return None if bool(keep.all()) else keep


def _continuation_mask(lens_before, past_len: int, q_len: int, keep, attention_mask, compress_v, device):
    """[B, 1, q, past_len + q] bool mask of a chunk of q new tokens over the
    decoded past of each sequence and the chunk itself.

    V-compressed layers store only a sequence's real tokens, so sequence b's
    past is the first lens_before[b] decoded positions: beyond them the rows
    hold this chunk's own tokens (stored before decoding) or zeros, and are
    hidden.  Within the chunk the mask is causal and hides padding tokens
    (``keep`` False) from every row but their own, so no row is empty.
    K-only layers keep every position in step with the base cache's V, so
    their past is masked by the model's own 4-D attention mask when it has
    one."""
    B = len(lens_before)
    causal = torch.ones(q_len, q_len, dtype=torch.bool, device=device).tril()
    if not compress_v:
        if attention_mask is not None and attention_mask.dim() == 4 and attention_mask.shape[-1] >= past_len + q_len:
            m = attention_mask[:, :, -q_len:, -(past_len + q_len):]
            return m if m.dtype == torch.bool else (m == 0)
        return torch.cat([torch.ones(q_len, past_len, dtype=torch.bool, device=device), causal], dim=1)
    lb = torch.tensor(lens_before, device=device)
    past_ok = (torch.arange(past_len, device=device)[None, :] < lb[:, None])[:, None, :].expand(B, q_len, past_len)
    new_ok = causal[None].expand(B, q_len, q_len)
    if keep is not None:
        eye = torch.eye(q_len, dtype=torch.bool, device=device)[None]
        new_ok = new_ok & (keep[:, None, :].to(torch.bool) | eye)
    return torch.cat([past_ok, new_ok], dim=2)[:, None]


def _probe_attention_module(module, config) -> dict:
    return {
        "is_cross_attention": bool(getattr(module, "is_cross_attention", False)),
        "has_fused_qkv": hasattr(module, "qkv_proj") or hasattr(module, "c_attn"),
        "has_separate_qkv": all(getattr(module, p, None) is not None for p in ("q_proj", "k_proj", "v_proj")),
        "sliding_window": getattr(module, "sliding_window", None) or getattr(config, "sliding_window", None),
        "attn_logit_softcapping": getattr(config, "attn_logit_softcapping", None),
        "rope_expected": _config_uses_rope(config),
    }


def _config_uses_rope(config) -> bool:
    for attr in ("rope_theta", "rope_scaling", "rope_parameters", "rotary_emb_base"):
        if getattr(config, attr, None) is not None:
            return True
    return getattr(config, "position_embedding_type", "rope") in ("rope", "rotary")


def make_fused_attention_forward(attn_module, cache: CompressedKVCache, quantizer: TurboQuantMSE,
                                 layer_idx: int, config=None, compress_v: bool = True):
    """Replacement forward for one decoder self-attention layer (reference
    ``hf/fused_cache.py:386-682``)."""
    if config is not None:
        probe = _probe_attention_module(attn_module, config)
        if probe["is_cross_attention"]:
            raise ValueError(f"Layer {layer_idx}: cross-attention layers cannot be patched")
        if probe["has_fused_qkv"] and not probe["has_separate_qkv"]:
            raise ValueError(f"Layer {layer_idx}: fused QKV projections are not supported")
        if probe["attn_logit_softcapping"] is not None:
            raise ValueError(f"Layer {layer_idx}: attention logit softcapping is not supported")
        if probe["sliding_window"] is not None:
            raise ValueError(f"Layer {layer_idx}: sliding-window attention is not supported")
    head_dim = quantizer.head_dim
    scale = float(getattr(attn_module, "scaling", None) or 1.0 / math.sqrt(head_dim))
    n_heads = attn_module.q_proj.out_features // head_dim
    n_kv_heads = attn_module.k_proj.out_features // head_dim
    n_rep = n_heads // n_kv_heads
    q_norm = getattr(attn_module, "q_norm", None)
    k_norm = getattr(attn_module, "k_norm", None)

    def fused_forward(hidden_states, position_embeddings=None, attention_mask=None,
                      past_key_values=None, cache_position=None, **kwargs):
        bsz, q_len, _ = hidden_states.size()
        q = attn_module.q_proj(hidden_states).view(bsz, q_len, n_heads, head_dim).transpose(1, 2)
        k = attn_module.k_proj(hidden_states).view(bsz, q_len, n_kv_heads, head_dim).transpose(1, 2)
        v = attn_module.v_proj(hidden_states).view(bsz, q_len, n_kv_heads, head_dim).transpose(1, 2)
        if q_norm is not None:
            q = q_norm(q)
        if k_norm is not None:
            k = k_norm(k)
        if position_embeddings is not None:
            cos, sin = position_embeddings
            q, k = _apply_rotary_pos_emb(q, k, cos, sin)

        lens_before = cache.seq_lens(layer_idx)  # per sequence, before this chunk is stored
        had_past = bool(lens_before) and max(lens_before) > 0
        past_len = max(lens_before) if had_past else 0
        # V-compressed layers drop masked-out (padding) tokens so each sequence's
        # pages hold only its own tokens; K-only layers keep every position so K
        # lines up with the full-precision V of the base cache, and mask instead
        keep = _keep_from_mask(attention_mask, q_len) if compress_v else None
        cache.store_compressed_kv(k, v, layer_idx, keep=keep)
        # sequence-length bookkeeping of the base class (one element per token)
        if compress_v:
            cache.update(k[..., :1], v[..., :1], layer_idx)
            raw_v = None
        else:
            _, raw_v = cache.update(k[..., :1], v, layer_idx)

        if q_len == 1 and compress_v:
            out = cache.decode_attention(q[:, :, 0], layer_idx, scale).unsqueeze(2)
        elif q_len == 1:
            # K-only layer (reference :591-624 with V uncompressed)
            kd = cache.decode_keys(layer_idx).to(q.dtype)
            S = kd.shape[2]
            scores = torch.matmul(q.float(), _repeat_kv(kd, n_rep).float().transpose(-1, -2)) * scale
            if attention_mask is not None and attention_mask.dim() == 4:
                m = attention_mask[:, :, -1:, -S:]
                scores = scores.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else scores + m.float()
            w = torch.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype)
            out = torch.matmul(w, _repeat_kv(raw_v[:, :, -S:], n_rep))
        elif not had_past:
            mask = attention_mask[:, :, :q_len, :q_len] if attention_mask is not None and attention_mask.dim() == 4 else None
            out = F.scaled_dot_product_attention(q, _repeat_kv(k, n_rep), _repeat_kv(v, n_rep),
                                                 attn_mask=mask, scale=scale, is_causal=mask is None)
        else:
            # new tokens attend over the decoded past and themselves (causal)
            kd = cache.decode_keys(layer_idx)[:, :, :past_len].to(q.dtype)
            vd = (cache.decode_values(layer_idx)[:, :, :past_len].to(q.dtype) if compress_v
                  else raw_v[:, :, :past_len])
            kk = torch.cat([kd, k], dim=2)
            vv = torch.cat([vd, v], dim=2)
            mask = _continuation_mask(lens_before, past_len, q_len, keep, attention_mask, compress_v, q.device)
            out = F.scaled_dot_product_attention(q, _repeat_kv(kk, n_rep), _repeat_kv(vv, n_rep),
                                                 attn_mask=mask, scale=scale)
        out = out.transpose(1, 2).reshape(bsz, q_len, -1)
        o_proj = getattr(attn_module, "o_proj", None) or getattr(attn_module, "out_proj", None)
        return o_proj(out), None

    return fused_forward


# --------------------------------------------------------------------------
# model-level entry points
# --------------------------------------------------------------------------

def _resolve_config(model):
    config = model.config
    return getattr(config, "text_config", config)


def _resolve_head_dim(config) -> int:
    hd = getattr(config, "head_dim", None)
    if hd:
        return hd
    hs, nh = getattr(config, "hidden_size", None), getattr(config, "num_attention_heads", None)
    return hs // nh if hs and nh else 0


def _is_full_attention_layer(module, name: str = "") -> bool:
    if getattr(module, "is_cross_attention", False):
        return False
    if any(kw in name.lower() for kw in _SKIP_NAME_KEYWORDS):
        return False
    has_qkv = all(getattr(module, p, None) is not None for p in ("q_proj", "k_proj", "v_proj"))
    return has_qkv and (hasattr(module, "o_proj") or hasattr(module, "out_proj"))


def check_model_compatibility(model) -> dict:
    """Whether ``patch_model`` can patch this model (reference :750-880)."""
    config = _resolve_config(model)
    head_dim = _resolve_head_dim(config)
    n_q = getattr(config, "num_attention_heads", 0)
    n_kv = getattr(config, "num_key_value_heads", n_q)
    issues, unsupported = [], []
    eligible = total = fused_qkv = cross = 0
    for name, module in model.named_modules():
        total += 1
        if getattr(module, "is_cross_attention", False):
            cross += 1
            continue
        if (hasattr(module, "qkv_proj") or hasattr(module, "c_attn")) and not all(
                hasattr(module, p) for p in ("q_proj", "k_proj", "v_proj")):
            fused_qkv += 1
        if _is_full_attention_layer(module, name):
            eligible += 1
    if head_dim not in (128, 256):
        issues.append(f"head_dim {head_dim} is not supported by the gfx950 paged kernels (128 or 256)")
    if n_kv > 0 and n_q % n_kv != 0:
        issues.append(f"n_q_heads ({n_q}) is not divisible by n_kv_heads ({n_kv})")
    elif n_kv > 0 and n_q // n_kv > 16:
        issues.append(f"GQA group {n_q // n_kv} exceeds 16")
    if eligible == 0:
        issues.append("No compatible attention layers found (need separate q/k/v and o projections)")
    if not _config_uses_rope(config):
        issues.append("Model config does not indicate RoPE usage")
    if getattr(config, "attn_logit_softcapping", None) is not None:
        unsupported.append("logit_softcapping")
    if getattr(config, "sliding_window", None) is not None:
        unsupported.append("sliding_window")
    if unsupported:
        issues.append(f"Unsupported attention features: {', '.join(unsupported)}")
    arch = type(model).__name__
    return {
        "compatible": not issues, "head_dim_valid": head_dim in (128, 256), "head_dim": head_dim,
        "n_q_heads": n_q, "n_kv_heads": n_kv, "eligible_layers": eligible, "total_layers": total,
        "issues": issues, "rope_detected": _config_uses_rope(config),
        "sliding_window": getattr(config, "sliding_window", None), "unsupported_features": unsupported,
        "fused_qkv_layers": fused_qkv, "cross_attention_layers": cross, "architecture": arch,
        "known_compatible": arch in KNOWN_COMPATIBLE,
    }


def _resolve_compress_v(compress_v, layer_idx: int, n_layers: int) -> bool:
    """Reference :964-980: True / False / "boundary" (first and last 2 layers
    keep V in full precision) / callable(layer_idx, n_layers)."""
    if callable(compress_v):
        return bool(compress_v(layer_idx, n_layers))
    if compress_v == "boundary":
        return not (layer_idx < 2 or layer_idx >= n_layers - 2)
    if isinstance(compress_v, bool):
        return compress_v
    raise ValueError(f"compress_v must be a bool, 'boundary' or a callable, got {compress_v!r}")


SMOKE_MIN_COSINE = 0.8  # reference hf/fused_cache.py:947


def _swap_forwards(model, forwards: dict) -> dict:
    """Install ``forwards`` (module name -> forward) and return the ones they replace."""
    replaced = {}
    for name, module in model.named_modules():
        if name in forwards:
            replaced[name] = module.forward
            module.forward = forwards[name]
    return replaced


def _smoke_test(model, cache: CompressedKVCache, originals: dict, config) -> float:
    """Verify the patched model against the unpatched one (reference
    ``hf/fused_cache.py:883-961``): a 4-token prompt and one decode step
    through the patched model (the step reads the compressed pages through
    the fused decode attention), then the same 5 tokens through the original
    forwards with no cache.  The cosine similarity of the two last-position
    logit vectors must reach 0.8, as in the reference; a fused forward that
    raises is reported the same way.  Returns the similarity; the model is
    left patched with an empty cache."""
    device = next(model.parameters()).device
    vocab = getattr(config, "vocab_size", 32000)
    ids = torch.randint(0, vocab, (1, 5), device=device)
    try:
        with torch.inference_mode():
            model(ids[:, :4], past_key_values=cache, use_cache=True)
            fused = model(ids[:, 4:], past_key_values=cache, use_cache=True).logits[0, -1].float()
    except Exception as exc:  # report as the reference does
        cache.reset()
        raise RuntimeError(f"Smoke test failed: fused forward raised {type(exc).__name__}: {exc}. "
                           "This model architecture may not be compatible with fused-turboquant; "
                           "see check_model_compatibility(model)") from exc
    cache.reset()
    patched = _swap_forwards(model, originals)
    try:
        with torch.inference_mode():
            ref = model(ids, use_cache=False).logits[0, -1].float()
    except Exception:  # the reference skips the check when its own forward fails
        logger.debug("Smoke test skipped: the unpatched forward failed")
        return float("nan")
    finally:
        _swap_forwards(model, patched)
    cos = torch.nn.functional.cosine_similarity(fused[None], ref[None]).item()
    if not math.isfinite(cos) or cos < SMOKE_MIN_COSINE:
        raise RuntimeError(f"Smoke test failed: cosine similarity between fused and reference logits is "
                           f"{cos:.4f} (threshold {SMOKE_MIN_COSINE}); the fused attention path is wrong "
                           f"for {type(model).__name__}. Pass verify=False to skip this check.")
    logger.info("Smoke test passed: logit cosine similarity = %.4f", cos)
    return cos


def patch_model(model, bits: int = 4, head_dim: int | None = None, verify: bool = True,
                compress_v: bool | str = True, max_iterations: int = 300, num_grid_points: int = 50000,
                strategy: str | None = None, target_compression: float | None = None,
                quality_target: float | None = None, tokenizer=None, calibration_text: str | None = None,
                quantizer_kind: str = "rht", v_bits: int | None = None,
                boundary_protect: int = 0) -> CompressedKVCache:
    """Patch every full-attention layer to store TurboQuant-compressed K/V and
    decode through the gfx950 kernels (reference ``hf/fused_cache.py:982-1270``).

    Returns the ``CompressedKVCache`` to pass as ``past_key_values``.
    ``quantizer_kind="planar"`` and ``strategy="adaptive"`` (research
    extensions of the reference) are not part of this build and raise.
    """
    if quantizer_kind != "rht":
        raise NotImplementedError(f"quantizer_kind={quantizer_kind!r}: only 'rht' is built on gfx950")
    if strategy is not None:
        raise NotImplementedError(f"strategy={strategy!r} (adaptive bit calibration) is not built")
    if bits not in (2, 3, 4):
        raise ValueError(f"bits must be 2, 3, or 4, got {bits}")
    if v_bits is None:
        v_bits = bits
    if v_bits not in (2, 3, 4):
        raise ValueError(f"v_bits must be 2, 3, or 4 (or None), got {v_bits}")
    if not isinstance(boundary_protect, int) or boundary_protect < 0:
        raise ValueError(f"boundary_protect must be a non-negative integer, got {boundary_protect!r}")

    config = _resolve_config(model)
    device = next(model.parameters()).device
    hd = head_dim if head_dim is not None else _resolve_head_dim(config)
    if hd not in (128, 256):
        raise ValueError(f"head_dim={hd}: the gfx950 paged kernels support head_dim 128 or 256")
    eligible = [(n, m) for n, m in model.named_modules() if _is_full_attention_layer(m, n)]
    n_layers = len(eligible)
    tqs: dict = {}

    def get_tq(b: int) -> TurboQuantMSE:
        if b not in tqs:
            tqs[b] = TurboQuantMSE(head_dim=hd, bits=b, device=device, max_iterations=max_iterations,
                                   num_grid_points=num_grid_points)
        return tqs[b]

    cache = CompressedKVCache(get_tq(bits), compress_v=compress_v is not False)
    n_boundary = min(boundary_protect, n_layers // 2)
    skip = set(range(n_boundary)) | set(range(n_layers - n_boundary, n_layers)) if n_boundary else set()
    originals = {}
    for pos, (name, module) in enumerate(eligible):
        if pos in skip:
            continue
        layer_idx = getattr(module, "layer_idx", pos)  # the index the base cache sees
        tq = get_tq(bits)
        cache.set_layer_quantizer(layer_idx, tq)
        if v_bits != bits:
            cache.set_layer_quantizer_v(layer_idx, get_tq(v_bits))
        originals[name] = module.forward
        module.forward = make_fused_attention_forward(
            module, cache, tq, layer_idx, config=config,
            compress_v=_resolve_compress_v(compress_v, pos, n_layers))
    model._fused_tq_originals = originals
    if not originals:
        logger.warning("No attention layers were patched; see check_model_compatibility(model)")
    elif verify:
        _smoke_test(model, cache, originals, config)
        cache.reset()
    return cache


def unpatch_model(model) -> None:
    """Restore the original attention forwards (reference :1273-1280)."""
    originals = getattr(model, "_fused_tq_originals", {})
    for name, module in model.named_modules():
        if name in originals:
            module.forward = originals[name]
    model._fused_tq_originals = {}


class FusedTurboQuantRunner:
    """Patch, generate, unpatch (reference :1283-1320)."""

    def __init__(self, model, tokenizer, bits: int = 4):
        self.model, self.tokenizer, self.bits = model, tokenizer, bits

    def generate(self, prompt: str, max_new_tokens: int = 200, do_sample: bool = False) -> str:
        cache = patch_model(self.model, bits=self.bits)
        inputs = self.tokenizer(prompt, return_tensors="pt").to(self.model.device)
        n_in = inputs["input_ids"].shape[-1]
        with torch.inference_mode():
            out = self.model.generate(**inputs, past_key_values=cache, max_new_tokens=max_new_tokens,
                                      do_sample=do_sample, use_cache=True)
        unpatch_model(self.model)
        return self.tokenizer.decode(out[0][n_in:], skip_special_tokens=True)
