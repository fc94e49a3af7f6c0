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

Head dims: 128 and 256 use the paged format and the fused paged decode
attention; any other power of two (Gemma 4's 512-wide global layers, for
example) keeps the reference's flat per-sequence rows of codes + fp16 norms,
encoded and decoded by the codec kernels, and attends with torch ops over
the decoded K / V -- as do sliding-window layers, whose decode step masks all
but the last ``sliding_window`` positions and the first ``sink_tokens``
(reference ``:600-611``).  Gemma 4's K = V layers (no ``v_proj``: V is the
k_proj output through ``v_norm``) and per-layer head dims are handled;
layers that share another layer's KV are refused (reference ``:421-426``).
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


class _LayerFlat:
    """Compressed K / V of one layer whose head dim has no paged kernel: per
    sequence a row of ``cap`` positions of codes [Hkv, cap, d * bits / 8] and
    fp16 norms [Hkv, cap] (the reference's flat CompressedTensor layout,
    ``hf/fused_cache.py:195-222``), grown by doubling; token i of sequence b
    sits at position i of row b."""

    def __init__(self, batch: int, hkv: int, d: int, k_tq: TurboQuantMSE, v_tq: TurboQuantMSE, device):
        self.B, self.hkv, self.d = batch, hkv, d
        self.k_tq, self.v_tq = k_tq, v_tq
        self.cap = 0
        self.kp = self.kn = self.vp = self.vn = None
        self.lens = [0] * batch
        self.lens_dev = torch.zeros(batch, dtype=torch.int32, device=device)
        self.device = device

    def _ensure(self, need: int) -> None:
        if need <= self.cap:
            return
        new = max(need, 2 * self.cap, 64)

        def grow(t, tail, dtype):
            fresh = torch.zeros(self.B, self.hkv, new, *tail, dtype=dtype, device=self.device)
            if t is not None:
                fresh[:, :, :self.cap] = t
            return fresh
        self.kp = grow(self.kp, (self.d * self.k_tq.bits // 8,), torch.uint8)
        self.kn = grow(self.kn, (), torch.float16)
        self.vp = grow(self.vp, (self.d * self.v_tq.bits // 8,), torch.uint8)
        self.vn = grow(self.vn, (), torch.float16)
        self.cap = new

    def append(self, key: torch.Tensor, value: torch.Tensor, keep: Optional[torch.Tensor]) -> None:
        B, hkv, q, d = key.shape
        if self.k_tq is self.v_tq and key.shape == value.shape and key.dtype == value.dtype:
            ck, cv = self.k_tq.encode_kv(key, value)  # one launch for K and V
        else:
            ck, cv = self.k_tq.encode(key), self.v_tq.encode(value)
        if keep is None:
            counts = [q] * B
            pos = torch.tensor(self.lens, device=self.device).view(-1, 1) + torch.arange(q, device=self.device)
            sel = torch.ones(B, q, dtype=torch.bool, device=self.device)
        else:
            sel = keep.to(torch.bool)
            counts = sel.sum(dim=1).tolist()
            pos = torch.tensor(self.lens, device=self.device).view(-1, 1) + sel.long().cumsum(dim=1) - 1
        self._ensure(max(L + c for L, c in zip(self.lens, counts)))
        b_idx = torch.arange(B, device=self.device).view(-1, 1).expand(B, q)[sel]
        p_idx = pos[sel]
        self.kp[b_idx, :, p_idx] = ck.indices.permute(0, 2, 1, 3)[sel]
        self.kn[b_idx, :, p_idx] = ck.norms.permute(0, 2, 1)[sel]
        self.vp[b_idx, :, p_idx] = cv.indices.permute(0, 2, 1, 3)[sel]
        self.vn[b_idx, :, p_idx] = cv.norms.permute(0, 2, 1)[sel]
        self.lens = [L + c for L, c in zip(self.lens, counts)]
        self.lens_dev.copy_(torch.tensor(self.lens, dtype=torch.int32))

    def flat(self):
        L = max(self.lens) if self.lens else 0
        return self.kp[:, :, :L], self.kn[:, :, :L], self.vp[:, :, :L], self.vn[:, :, :L]


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
    def _layer(self, layer_idx: int, like: torch.Tensor):
        lp = self._pages.get(layer_idx)
        if lp is None:
            B, hkv, _, d = like.shape
            kind = _LayerPages if d in (128, 256) else _LayerFlat  # the paged kernels take 128 and 256
            lp = kind(B, hkv, d, self.get_layer_quantizer(layer_idx), self.get_layer_quantizer_v(layer_idx),
                      like.device)
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

    def decode_attention(self, query: torch.Tensor, layer_idx: int, scale: float,
                         sliding_window: Optional[int] = None, sink_tokens: int = 0) -> torch.Tensor:
        """query [B, Hq, d] -> [B, Hq, d] (query dtype): the fused paged decode
        attention; for flat (non-paged) layers and sliding windows, softmax
        attention in fp32 over the decoded K / V of each sequence's positions
        (with a window: the last ``sliding_window`` and the first
        ``sink_tokens``, reference ``hf/fused_cache.py:600-611``)."""
        lp = self._pages[layer_idx]
        if isinstance(lp, _LayerPages) and sliding_window is None:
            return P.paged_decode_attention(query, lp.kv_cache, lp.block_table, lp.lens_dev, lp.k_tq, lp.v_tq,
                                            scale=scale, max_seq_len=max(lp.lens))
        kd = self.decode_keys(layer_idx)
        vd = self.decode_values(layer_idx)
        B, hq, d = query.shape
        n_rep = hq // kd.shape[1]
        S = kd.shape[2]
        scores = torch.matmul(query.float().unsqueeze(2), _repeat_kv(kd, n_rep).transpose(-1, -2).contiguous())
        scores = scores * scale  # [B, Hq, 1, S]
        pos = torch.arange(S, device=query.device).view(1, -1)
        lens = lp.lens_dev.view(-1, 1).to(torch.int64)
        ok = pos < lens
        if sliding_window is not None:
            ok = ok & ((pos >= lens - sliding_window) | (pos < sink_tokens))
        scores = scores.masked_fill(~ok[:, None, None, :], float("-inf"))
        w = torch.softmax(scores, dim=-1)
        w = torch.nan_to_num(w, nan=0.0)  # a sequence with no positions gives 0
        return torch.matmul(w, _repeat_kv(vd, n_rep)).squeeze(2).to(query.dtype)

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


def _keep_from_mask(attention_mask, q_len: int, window: Optional[int] = None) -> Optional[torch.Tensor]:
    """[B, q] bool of the new tokens that are not padding, or None when none
    is.  Token j is read from query row r_j = min(j + window - 1, q - 1), the
    last row whose window still holds it (the last row without a window):
    a real token is visible there, a padding token is not."""
    if attention_mask is None or attention_mask.dim() != 4:
        return None
    m = attention_mask[:, 0, -q_len:, -q_len:]
    vis = m if m.dtype == torch.bool else (m == 0)
    j = torch.arange(q_len, device=vis.device)
    r = torch.full_like(j, q_len - 1) if window is None else torch.clamp(j + window - 1, max=q_len - 1)
    keep = vis[:, r, j]
    return None if bool(keep.all()) else keep


def _continuation_mask(lens_before, past_len: int, q_len: int, keep, attention_mask, compress_v, device,
                       window: Optional[int] = None):
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
    if window is not None:
        # row i of sequence b sits at position lens_before[b] + (its index among
        # the kept tokens); it sees the positions within `window` of itself
        kept = (keep.to(torch.long) if keep is not None else torch.ones(B, q_len, dtype=torch.long, device=device))
        row_pos = lb[:, None] + kept.cumsum(dim=1) - 1                             # [B, q]
        past_pos = torch.arange(past_len, device=device)[None, None, :]
        past_ok = past_ok & (past_pos > row_pos[:, :, None] - window)
        new_pos = lb[:, None] + kept.cumsum(dim=1) - 1
        new_ok = new_ok & (new_pos[:, None, :] > row_pos[:, :, None] - window)
    return torch.cat([past_ok, new_ok], dim=2)[:, None]


def _module_k_eq_v(module) -> bool:
    """Gemma 4 full-attention layers (``attention_k_eq_v``): no ``v_proj``, V
    is the k_proj output through ``v_norm`` (reference ``:89-105``)."""
    has_qk = getattr(module, "q_proj", None) is not None and getattr(module, "k_proj", None) is not None
    if not has_qk or getattr(module, "v_proj", "missing") is not None:
        return False
    return bool(getattr(module, "use_alternative_attention", False)) or bool(
        getattr(getattr(module, "config", None), "attention_k_eq_v", False))


def _module_is_kv_shared(module) -> bool:
    """Gemma 4 layers that reuse another layer's K / V (reference ``:108-110``)."""
    return bool(getattr(module, "is_kv_shared_layer", False))


def _layer_sliding_window(module, config) -> Optional[int]:
    """The module's own window when it declares one (None on Gemma's full
    layers), else the config's."""
    if hasattr(module, "sliding_window"):
        return getattr(module, "sliding_window")
    return _cfg(config, "sliding_window", None) if config is not None else None


def _probe_attention_module(module, config) -> dict:
    k_eq_v = _module_k_eq_v(module)
    has_qkv = (getattr(module, "q_proj", None) is not None and getattr(module, "k_proj", None) is not None
               and (getattr(module, "v_proj", None) is not None or k_eq_v))
    return {
        "is_cross_attention": bool(getattr(module, "is_cross_attention", False)),
        "has_fused_qkv": hasattr(module, "qkv_proj") or hasattr(module, "c_attn"),
        "has_separate_qkv": has_qkv,
        "k_eq_v": k_eq_v,
        "is_kv_shared": _module_is_kv_shared(module),
        "sliding_window": _layer_sliding_window(module, config),
        "attn_logit_softcapping": _cfg(config, "attn_logit_softcapping", None),
        "rope_expected": _config_uses_rope(config),
    }


def _config_uses_rope(config) -> bool:
    for attr in ("rope_theta", "rope_scaling", "rope_parameters", "rotary_emb_base"):
        if _cfg(config, attr, None) is not None:
            return True
    return _cfg(config, "position_embedding_type", "rope") in ("rope", "rotary")


def make_fused_attention_forward(attn_module, cache: CompressedKVCache, quantizer: TurboQuantMSE,
                                 layer_idx: int, config=None, compress_v: bool = True):
    """Replacement forward for one decoder self-attention layer (reference
    ``hf/fused_cache.py:386-682``)."""
    k_eq_v = _module_k_eq_v(attn_module)
    window = _layer_sliding_window(attn_module, config)
    if config is not None:
        probe = _probe_attention_module(attn_module, config)
        if probe["is_cross_attention"]:
            raise ValueError(f"Layer {layer_idx}: cross-attention layers cannot be patched")
        if probe["is_kv_shared"]:
            raise ValueError(f"Layer {layer_idx}: a KV-shared layer (is_kv_shared_layer=True) reuses another "
                             "layer's K/V and cannot be patched")
        if probe["has_fused_qkv"] and not probe["has_separate_qkv"]:
            raise ValueError(f"Layer {layer_idx}: fused QKV projections are not supported")
        if probe["attn_logit_softcapping"] is not None:
            raise ValueError(f"Layer {layer_idx}: attention logit softcapping is not supported")
    head_dim = quantizer.head_dim
    scaling = getattr(attn_module, "scaling", None)  # Gemma sets 1.0 (Q and K are RMS-normalised)
    scale = float(scaling) if scaling is not None else 1.0 / math.sqrt(head_dim)
    n_heads = attn_module.q_proj.out_features // head_dim
    n_kv_heads = attn_module.k_proj.out_features // head_dim
    n_rep = n_heads // n_kv_heads
    q_norm = getattr(attn_module, "q_norm", None)
    k_norm = getattr(attn_module, "k_norm", None)
    v_norm = getattr(attn_module, "v_norm", None)
    n_sink = int(_cfg(config, "sink_tokens", 4) or 0) if config is not None else 4

    def fused_forward(hidden_states, position_embeddings=None, attention_mask=None,
                      past_key_values=None, cache_position=None, **kwargs):
        bsz, q_len, _ = hidden_states.size()
        q = attn_module.q_proj(hidden_states).view(bsz, q_len, n_heads, head_dim).transpose(1, 2)
        k_out = attn_module.k_proj(hidden_states)
        v_out = k_out if (k_eq_v or getattr(attn_module, "v_proj", None) is None) else attn_module.v_proj(hidden_states)
        k = k_out.view(bsz, q_len, n_kv_heads, head_dim).transpose(1, 2)
        v = v_out.view(bsz, q_len, n_kv_heads, head_dim).transpose(1, 2)
        if q_norm is not None:
            q = q_norm(q)
        if k_norm is not None:
            k = k_norm(k)
        if v_norm is not None:  # V takes no RoPE; Gemma normalises it on its own
            v = v_norm(v)
        if position_embeddings is not None:
            cos, sin = position_embeddings
            q, k = _apply_rotary_pos_emb(q, k, cos, sin)

        lens_before = cache.seq_lens(layer_idx)  # per sequence, before this chunk is stored
        had_past = bool(lens_before) and max(lens_before) > 0
        past_len = max(lens_before) if had_past else 0
        # V-compressed layers drop masked-out (padding) tokens so each sequence's
        # pages hold only its own tokens; K-only layers keep every position so K
        # lines up with the full-precision V of the base cache, and mask instead
        keep = _keep_from_mask(attention_mask, q_len, window) if compress_v else None
        cache.store_compressed_kv(k, v, layer_idx, keep=keep)
        # sequence-length bookkeeping of the base class (one element per token)
        if compress_v:
            cache.update(k[..., :1], v[..., :1], layer_idx)
            raw_v = None
        else:
            _, raw_v = cache.update(k[..., :1], v, layer_idx)

        if q_len == 1 and compress_v:
            out = cache.decode_attention(q[:, :, 0], layer_idx, scale, sliding_window=window,
                                         sink_tokens=n_sink).unsqueeze(2)
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
            if mask is None and window is not None and q_len > window:  # causal within the window
                i = torch.arange(q_len, device=q.device)
                mask = (i[None, :] <= i[:, None]) & (i[None, :] > i[:, None] - window)
            out = F.scaled_dot_product_attention(q, _repeat_kv(k, n_rep), _repeat_kv(v, n_rep),
                                                 attn_mask=mask, scale=scale, is_causal=mask is None)
        else:
            # new tokens attend over the decoded past and themselves (causal)
            kd = cache.decode_keys(layer_idx)[:, :, :past_len].to(q.dtype)
            vd = (cache.decode_values(layer_idx)[:, :, :past_len].to(q.dtype) if compress_v
                  else raw_v[:, :, :past_len])
            kk = torch.cat([kd, k], dim=2)
            vv = torch.cat([vd, v], dim=2)
            mask = _continuation_mask(lens_before, past_len, q_len, keep, attention_mask, compress_v, q.device,
                                      window)
            out = F.scaled_dot_product_attention(q, _repeat_kv(kk, n_rep), _repeat_kv(vv, n_rep),
                                                 attn_mask=mask, scale=scale)
        out = out.transpose(1, 2).reshape(bsz, q_len, -1)
        o_proj = getattr(attn_module, "o_proj", None) or getattr(attn_module, "out_proj", None)
        return o_proj(out), None

    return fused_forward


# --------------------------------------------------------------------------
# model-level entry points
# --------------------------------------------------------------------------

def _cfg(config, name: str, default=None):
    """A config attribute, or ``default`` when it is missing or, on a
    heterogeneous (per-layer) config such as Gemma 4's, not defined globally."""
    try:
        return getattr(config, name, default)
    except Exception:  # transformers refuses global reads of per-layer attributes
        return default


def _resolve_config(model):
    config = model.config
    return _cfg(config, "text_config", config)


def _resolve_head_dim(config) -> int:
    hd = _cfg(config, "head_dim", None)
    if hd:
        return hd
    hs, nh = _cfg(config, "hidden_size", None), _cfg(config, "num_attention_heads", None)
    return hs // nh if hs and nh else 0


def _resolve_layer_head_dim(module, config) -> int:
    """The layer's own head_dim when the module declares one (Gemma 4: 256 on
    sliding layers, 512 on full ones), else the config's (reference
    ``:728-740``)."""
    hd = getattr(module, "head_dim", None)
    return hd if isinstance(hd, int) and hd > 0 else _resolve_head_dim(config)


def _is_full_attention_layer(module, name: str = "") -> bool:
    """A decoder self-attention module this library can patch: separate q / k
    projections, a v projection or K = V (Gemma 4), an output projection; not
    cross-attention, not a vision tower, not a KV-shared layer (reference
    ``:686-707``)."""
    if getattr(module, "is_cross_attention", False) or _module_is_kv_shared(module):
        return False
    if any(kw in name.lower() for kw in _SKIP_NAME_KEYWORDS):
        return False
    has_qk = all(getattr(module, p, None) is not None for p in ("q_proj", "k_proj"))
    has_v = getattr(module, "v_proj", None) is not None or _module_k_eq_v(module)
    return has_qk and has_v and (hasattr(module, "o_proj") or hasattr(module, "out_proj"))


def _head_dim_ok(hd: int) -> bool:
    return 8 <= hd <= 4096 and (hd & (hd - 1)) == 0


def check_model_compatibility(model) -> dict:
    """Whether ``patch_model`` can patch this model (reference :750-880).

    Per-layer head dims are read from the attention modules; each must be a
    power of two in [8, 4096] (128 and 256 take the fused paged decode, the
    others torch attention over the decoded cache).  Sliding-window layers
    are supported; logit soft-capping and KV-shared layers are not."""
    config = _resolve_config(model)
    head_dim = _resolve_head_dim(config)
    n_q = _cfg(config, "num_attention_heads", 0)
    n_kv = _cfg(config, "num_key_value_heads", n_q) or n_q
    issues, unsupported = [], []
    eligible = total = fused_qkv = cross = kv_shared = k_eq_v = 0
    layer_hds = []
    for name, module in model.named_modules():
        total += 1
        if getattr(module, "is_cross_attention", False):
            cross += 1
            continue
        if _module_is_kv_shared(module):
            kv_shared += 1
            continue
        if (hasattr(module, "qkv_proj") or hasattr(module, "c_attn")) and not all(
                hasattr(module, p) for p in ("q_proj", "k_proj", "v_proj")):
            fused_qkv += 1
        if _is_full_attention_layer(module, name):
            eligible += 1
            k_eq_v += int(_module_k_eq_v(module))
            hd_l = _resolve_layer_head_dim(module, config)
            layer_hds.append(hd_l)
            if hd_l > 0:
                nq_l, nkv_l = module.q_proj.out_features // hd_l, module.k_proj.out_features // hd_l
                if nkv_l <= 0 or nq_l % nkv_l or nq_l // nkv_l > 16:
                    issues.append(f"{name}: {nq_l} query heads over {nkv_l} kv heads (need a group of <= 16)")
    hds = sorted(set(layer_hds)) or ([head_dim] if head_dim else [])
    bad = [hd for hd in hds if not _head_dim_ok(hd)]
    if bad:
        issues.append(f"head_dim {bad} is not a power of two in [8, 4096]")
    if n_kv > 0 and n_q % n_kv != 0:
        issues.append(f"n_q_heads ({n_q}) is not divisible by n_kv_heads ({n_kv})")
    elif n_kv > 0 and n_q // n_kv > 16:
        issues.append(f"GQA group {n_q // n_kv} exceeds 16")
    if eligible == 0:
        issues.append("No compatible attention layers found (need separate q/k/v and o projections)")
    if kv_shared:
        issues.append(f"{kv_shared} KV-shared layers reuse another layer's K/V; they cannot be patched")
    if not _config_uses_rope(config):
        issues.append("Model config does not indicate RoPE usage")
    if _cfg(config, "attn_logit_softcapping", None) is not None:
        unsupported.append("logit_softcapping")
    if unsupported:
        issues.append(f"Unsupported attention features: {', '.join(unsupported)}")
    arch = type(model).__name__
    return {
        "compatible": not issues, "head_dim_valid": not bad, "head_dim": hds[0] if hds else head_dim,
        "head_dims": hds, "paged_head_dims": [hd for hd in hds if hd in (128, 256)],
        "n_q_heads": n_q, "n_kv_heads": n_kv, "eligible_layers": eligible, "total_layers": total,
        "issues": issues, "rope_detected": _config_uses_rope(config),
        "sliding_window": _cfg(config, "sliding_window", None), "unsupported_features": unsupported,
        "fused_qkv_layers": fused_qkv, "cross_attention_layers": cross, "kv_shared_layers": kv_shared,
        "k_eq_v_layers": k_eq_v, "architecture": arch, "known_compatible": arch in KNOWN_COMPATIBLE,
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
    shared = [n for n, m in model.named_modules() if _module_is_kv_shared(m)]
    if shared:
        raise ValueError(f"{len(shared)} KV-shared layers (e.g. {shared[0]}) reuse another layer's K/V, which "
                         "this cache keeps compressed; models with num_kv_shared_layers=0 can be patched")
    eligible = [(n, m) for n, m in model.named_modules() if _is_full_attention_layer(m, n)]
    n_layers = len(eligible)
    layer_hd = {n: (head_dim if head_dim is not None else _resolve_layer_head_dim(m, config)) for n, m in eligible}
    for n, hd in layer_hd.items():
        if not _head_dim_ok(hd):
            raise ValueError(f"head_dim={hd} ({n}): the gfx950 kernels take powers of two in [8, 4096]")
    tqs: dict = {}

    def get_tq(hd: int, b: int) -> TurboQuantMSE:
        if (hd, b) not in tqs:
            tqs[hd, b] = TurboQuantMSE(head_dim=hd, bits=b, device=device, max_iterations=max_iterations,
                                       num_grid_points=num_grid_points)
        return tqs[hd, b]

    hd0 = layer_hd[eligible[0][0]] if eligible else (head_dim or _resolve_head_dim(config))
    if not _head_dim_ok(hd0):
        raise ValueError(f"head_dim={hd0}: the gfx950 kernels take powers of two in [8, 4096]")
    cache = CompressedKVCache(get_tq(hd0, bits), compress_v=compress_v is not False)
    n_boundary = min(boundary_protect, n_layers // 2)
    skip = set(range(n_boundary)) | set(range(n_layers - n_boundary, n_layers)) if n_boundary else set()
    originals = {}
    for pos, (name, module) in enumerate(eligible):
        if pos in skip:
            continue
        layer_idx = getattr(module, "layer_idx", pos)  # the index the base cache sees
        tq = get_tq(layer_hd[name], bits)
        cache.set_layer_quantizer(layer_idx, tq)
        if v_bits != bits:
            cache.set_layer_quantizer_v(layer_idx, get_tq(layer_hd[name], v_bits))
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
