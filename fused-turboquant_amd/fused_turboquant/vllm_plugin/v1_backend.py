"""vLLM v1 ``TURBOQUANT`` attention backend on the gfx950 kernels
(reference ``vllm_plugin/v1_backend.py:120-1866``, ``kind=rht``).

The class surface is vLLM's (``AttentionBackend`` / ``AttentionImpl``
methods, the Impl ``__init__`` signature, ``do_kv_cache_update`` and
``forward`` over vLLM's metadata fields).  The classes derive from vLLM's
bases when vLLM is importable and stand alone otherwise, so the backend can
be driven directly (the tests feed it plain metadata objects).

Per call:

* ``do_kv_cache_update`` -> ``ftq_v1_store`` (K: norm, Hadamard, midpoint
  search, pack, fp16 norm; V: optional rotation, min/max uniform quant), the
  reference's ``_launch_store`` (``:712-749``).
* decode tokens -> ``ftq_v1_decode_attention`` (query rotation, split-K
  attention over the packed slots with norm correction, LSE merge, V
  un-rotation, output cast), the reference's ``_decode_attention*``
  (``:842-1093``).
* prefill of fresh sequences -> SDPA over the full-precision K/V of the
  batch, grouped K/V (``enable_gqa``, ``:1355-1358``), one launch per run of
  consecutive fresh sequences of one length (the reference uses flash-attn
  varlen there, ``:1283-1443``).
* prefill continuing a cached sequence -> the decode kernel with one
  synthetic sequence per query token (seq_len = cached + i + 1, same block
  table row): causal attention over the stored slots, the reference's
  continuation path (``:1359-1384``).

Boundary-protection layers (a plain cache dtype such as ``"auto"``; reference
``:335-366``) follow ``TURBOQUANT_BOUNDARY_PROTECT``: ``fp16`` stores raw fp16
K|V slots (``ftq_raw_store``, the reference's ``_store_raw_kv``, ``:1449-1505``)
and decodes them with ``ftq_raw_decode_attention`` (the reference's
``boundary_fp16_decode_attention``, ``triton_boundary_attn.py:28-219``); 2/3/4/8
run the TurboQuant path at that width inside the fp16-sized slot (8: 256
Lloyd-Max centroids for K, 8-bit uniform V), and ``fp8`` stores fp8 e4m3fn
keys with 8-bit uniform values (``boundary_tq_config.py``).

Sliding-window layers (``sliding_window=W``, vLLM's window: a query at
position p sees keys p - W + 1 .. p) decode from ``kv_start = max(0, seq_len
- W)`` per row, continuation rows likewise, and fresh prefill masks each
query block to its window.  The reference stores the window and attends the
whole context (``:316``); logit soft-capping, which it also stores without
applying (``:318``), is refused here.

Head sizes 64, 128 and 256.  At 128 with 2-4 bit codes decode runs on the
matrix-core kernels; every other head size and width (1-bit, 8-bit, fp8
keys) runs the fp32 decode kernel.

Deferred prefill (``TURBOQUANT_DEFER_PREFILL=1``, TurboQuant layers; reference
``:331-332``, ``:673-686``, ``:1095-1277``): a prefill store of 1 < N <=
capacity tokens skips the quantised store and writes the tokens as fp16 into
one per-layer prefix buffer (raw slots, positions 0..N-1); decode tokens then
run phase 1 = ``ftq_raw_decode_attention_lse`` over the prefix (sequence 0
only, as the reference's cu_seqlens [0, P, P, ...] give), phase 2 =
``ftq_v1_decode_attention_lse`` over positions [P, seq_len) of every
sequence, and a log-sum-exp merge of the two.  As in the reference, the
prefix length starts at 1 (one zero K/V row) until a prefill is deferred.
The capacity is vLLM's max(max_model_len, max_num_batched_tokens), or
``TURBOQUANT_DEFER_PREFILL_CAPACITY`` (default 32768) without vLLM.

Per-layer state (sorted centroids, midpoints) is cached on the ``layer``
object, like the reference's ``setup_layer`` (``rotation/matrix.py:34-42``).
The centroid table of vLLM's ``get_centroids`` is not available here; this
library's Lloyd-Max levels for (head_size, key bits) are used, and a table
vLLM attached as ``layer._tq_centroids`` with the right size takes precedence.
"""
from __future__ import annotations

import math
import os
from typing import Any, ClassVar, Optional

import torch
import torch.nn.functional as F

from .. import raw as RAW
from .. import v1 as V1
from .plugin import TQ_PRESETS, boundary_protect_enabled, boundary_protect_mode, env_flag, host_preset

# TURBOQUANT_KIND values the reference registers (vllm_plugin/rotation/*.py register_rotation)
ROTATION_KINDS = ("rht", "planar", "rotor", "iso_fast", "iso_full")

try:  # vLLM's base classes when present (not installed in every environment)
    from vllm.attention.backends.abstract import AttentionBackend as _BackendBase  # type: ignore
    from vllm.attention.backends.abstract import AttentionImpl as _ImplBase  # type: ignore
except Exception:  # pragma: no cover - depends on the environment
    _BackendBase = object
    _ImplBase = object


def _max_kv_splits() -> int:
    """Split-K factor of decode steps under CUDA/HIP graph capture, fixed so
    the captured launches and buffers do not depend on the step's context
    length: vLLM's attention_config.tq_max_kv_splits_for_cuda_graph
    (reference :569-574), else TURBOQUANT_MAX_KV_SPLITS (default 32)."""
    try:
        from vllm.config import get_current_vllm_config  # type: ignore
        v = int(get_current_vllm_config().attention_config.tq_max_kv_splits_for_cuda_graph)
    except Exception:
        v = int(os.environ.get("TURBOQUANT_MAX_KV_SPLITS", "32"))
    if not 1 <= v <= 1024:
        raise ValueError("the maximum KV split count must be in [1, 1024]")
    return v


def _buf(layer, name: str, shape: tuple, dtype, device) -> torch.Tensor:
    """A per-layer scratch tensor cached on the layer (reference
    _get_or_alloc_buf, v1_backend.py:1851-1866): allocated when first needed
    or when a larger one is, else the same storage, so decode steps allocate
    nothing after warm-up and captured graphs keep their addresses."""
    bufs = getattr(layer, "_fused_tq_bufs", None)
    if bufs is None:
        bufs = {}
        try:
            layer._fused_tq_bufs = bufs
        except AttributeError:  # a layer object that takes no attributes: cache on the Impl's side
            bufs = _buf.__dict__.setdefault("_fallback", {}).setdefault(id(layer), {})
    n = 1
    for x in shape:
        n *= int(x)
    t = bufs.get(name)
    if t is None or t.numel() < n or t.dtype != dtype or t.device != torch.device(device):
        t = torch.empty(max(n, 1), dtype=dtype, device=device)
        bufs[name] = t
    return t[:n].view(shape)


def _defer_capacity() -> int:
    """Positions of the deferred-prefill buffer: vLLM's max(max_model_len,
    max_num_batched_tokens) (reference :575-585), else
    TURBOQUANT_DEFER_PREFILL_CAPACITY (default 32768)."""
    try:
        from vllm.config import get_current_vllm_config  # type: ignore
        cfg = get_current_vllm_config()
        sched = getattr(cfg, "scheduler_config", None)
        mb = int(getattr(sched, "max_num_batched_tokens", 0) or 0) if sched is not None else 0
        return max(int(cfg.model_config.max_model_len), mb)
    except Exception:
        v = int(os.environ.get("TURBOQUANT_DEFER_PREFILL_CAPACITY", "32768"))
        if v < 2:
            raise ValueError("TURBOQUANT_DEFER_PREFILL_CAPACITY must be at least 2")
        return v


class FusedTurboQuantV1Backend(_BackendBase):
    """Backend class vLLM resolves from ``attention_backend="TURBOQUANT"``."""

    accept_output_buffer: bool = True
    forward_includes_kv_cache_update: bool = False
    supported_dtypes: ClassVar[list] = [torch.float16, torch.bfloat16]
    supported_kv_cache_dtypes: ClassVar[list] = [
        "auto", "float16", "bfloat16", "turboquant_4bit_nc", "turboquant_k3v4_nc", "turboquant_3bit_nc",
    ]

    @staticmethod
    def get_supported_kernel_block_sizes():
        return [16, 32, 64, 128]

    @staticmethod
    def get_name() -> str:
        return "TURBOQUANT"

    @staticmethod
    def get_impl_cls():
        return FusedTurboQuantV1Impl

    @staticmethod
    def get_builder_cls():
        from vllm.v1.attention.backends.turboquant_attn import TurboQuantMetadataBuilder  # type: ignore
        return TurboQuantMetadataBuilder

    @staticmethod
    def _slot_size_for(head_size: int, cache_dtype_str: Optional[str]) -> int:
        """Last-dim size: the preset's slot bytes (at least 2*head_size bf16
        elements when boundary layers share the allocation), rounded up to a
        power of two (reference ``v1_backend.py:171-209``)."""
        if isinstance(cache_dtype_str, str) and cache_dtype_str.startswith("turboquant_"):
            preset, _, _ = host_preset(cache_dtype_str)
            pk, pv = TQ_PRESETS[preset]
            return V1.slot_size(head_size, pk, pv, boundary_protect=boundary_protect_enabled())
        raw = 2 * head_size
        return 1 << (raw - 1).bit_length()

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                           cache_dtype_str: str = "turboquant_4bit_nc") -> tuple:
        slot = FusedTurboQuantV1Backend._slot_size_for(head_size, cache_dtype_str)
        return (num_blocks, block_size, num_kv_heads, slot)

    @classmethod
    def supports_kv_cache_dtype(cls, kv_cache_dtype) -> bool:
        if kv_cache_dtype is None:
            return True
        if kv_cache_dtype in cls.supported_kv_cache_dtypes:
            return True
        try:
            host_preset(kv_cache_dtype)
            return True
        except (ValueError, TypeError):
            return False

    @classmethod
    def supports_head_size(cls, head_size: int) -> bool:
        # 128: matrix-core decode for 2-4 bit codes; 64 and 256 (and every
        # other width): the fp32 decode kernel
        return head_size in (64, 128, 256)

    @classmethod
    def supports_compute_capability(cls, capability) -> bool:
        return True

    @classmethod
    def supports_sink(cls) -> bool:
        return False

    @staticmethod
    def use_cascade_attention(*args, **kwargs) -> bool:
        return False


class FusedTurboQuantV1Impl(_ImplBase):
    """Per-layer attention implementation (reference ``v1_backend.py:292-1866``)."""

    accept_output_buffer: bool = True
    supports_quant_query_input: bool = False

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int,
                 alibi_slopes: Optional[list] = None, sliding_window: Optional[int] = None,
                 kv_cache_dtype: str = "auto", logits_soft_cap: Optional[float] = None,
                 attn_type=None, kv_sharing_target_layer_name: Optional[str] = None, **kwargs: Any) -> None:
        if alibi_slopes is not None:
            raise NotImplementedError("ALiBi attention is not supported")
        if kv_sharing_target_layer_name is not None:
            raise NotImplementedError("KV sharing is not yet supported")
        if sliding_window is not None and int(sliding_window) <= 0:
            raise ValueError(f"sliding_window must be a positive token count, got {sliding_window}")
        if logits_soft_cap is not None:
            # the reference stores the value and never applies it (v1_backend.py:318); scores
            # here are not capped either, so a model that needs the cap is refused up front
            raise NotImplementedError("logit soft-capping is not supported by the TURBOQUANT backend")
        # Boundary-protection layers arrive with a plain cache dtype ("auto",
        # "float16", "bfloat16"; reference v1_backend.py:335-366): raw fp16
        # slots in mode "fp16", TurboQuant codes at N bits in mode N.
        is_boundary = not (isinstance(kv_cache_dtype, str) and kv_cache_dtype.startswith("turboquant_"))
        mode = boundary_protect_mode()
        self._is_raw = False
        self.key_fp8 = False
        if is_boundary:
            if mode == "fp16":
                self._is_raw = True
                self.preset, self.key_bits, self.value_bits = "raw_fp16", 16, 16
            elif mode in (2, 3, 4, 8):
                # N-bit Lloyd-Max keys and N-bit uniform values in the fp16-sized slot
                # (reference BoundaryTurboQuantConfig, boundary_tq_config.py)
                self.preset, self.key_bits, self.value_bits = f"boundary_{mode}bit", mode, mode
            elif mode == "fp8":
                # fp8 e4m3fn keys (no codebook, no norm) and 8-bit uniform values
                self.preset, self.key_bits, self.value_bits = "boundary_fp8", 8, 8
                self.key_fp8 = True
            else:
                raise NotImplementedError(f"kv_cache_dtype={kv_cache_dtype!r} needs a turboquant_* cache dtype "
                                          "when TURBOQUANT_BOUNDARY_PROTECT is off")
        else:
            self.preset, self.key_bits, self.value_bits = host_preset(kv_cache_dtype)
        if head_size not in (64, 128, 256):
            raise NotImplementedError("the gfx950 kernels support head_size 64, 128 and 256")
        group_limit = 8 if (self._is_raw and head_size == 128) else 16
        if num_heads % num_kv_heads != 0 or num_heads // num_kv_heads > group_limit:
            raise ValueError(f"num_heads must be a multiple of num_kv_heads with a group of at most {group_limit}")
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads
        self.num_kv_groups = num_heads // num_kv_heads
        # vLLM's window: a query at position p attends keys p - W + 1 .. p (flash-attn
        # window_size (W - 1, 0)); decode rows start at max(0, seq_len - W)
        self.sliding_window = int(sliding_window) if sliding_window is not None else None
        self.logits_soft_cap = logits_soft_cap
        self.kv_cache_dtype = kv_cache_dtype
        self.v_rotate = not self._is_raw and (env_flag("TURBOQUANT_V_ROTATE") or env_flag("TURBOQUANT_V_LLOYD_MAX"))
        self.defer_prefill = not self._is_raw and env_flag("TURBOQUANT_DEFER_PREFILL")
        if self.defer_prefill and self.sliding_window is not None:
            raise NotImplementedError("TURBOQUANT_DEFER_PREFILL with sliding-window layers is not supported")
        self._prefix_capacity = _defer_capacity() if self.defer_prefill else 0
        self.max_kv_splits = _max_kv_splits()
        # Lloyd-Max V codes (4-bit V; other widths stay uniform but rotated, as in the reference)
        self.v_lloyd_max = not self._is_raw and env_flag("TURBOQUANT_V_LLOYD_MAX")
        # rotation strategy (reference v1_backend.py:516-523): rht, or one of the block-diagonal
        # strategies (planar, rotor, iso_fast, iso_full) applied inside the store / decode /
        # merge kernels.  Names are matched as given, like the reference's registry lookup.
        self.kind = os.environ.get("TURBOQUANT_KIND", "rht")
        if not self._is_raw and self.kind not in ROTATION_KINDS:
            raise ValueError(f"TURBOQUANT_KIND={self.kind!r} not registered. Pick one of "
                             f"{', '.join(ROTATION_KINDS)}")

    # -- per-layer state ---------------------------------------------------
    def _state(self, layer, device) -> V1.TurboQuantV1Layer:
        st = getattr(layer, "_fused_tq_state", None)
        if st is None or st.centroids.device != torch.device(device):
            cent = getattr(layer, "_tq_centroids", None)
            if cent is not None and cent.numel() != (1 << self.key_bits):
                cent = None
            st = V1.TurboQuantV1Layer(self.head_size, self.key_bits, self.value_bits,
                                      v_rotate=self.v_rotate, centroids=cent, device=device,
                                      v_lloyd_max=self.v_lloyd_max, kind=self.kind, key_fp8=self.key_fp8)
            layer._fused_tq_state = st
        return st

    def _prefix(self, layer, device):
        """The deferred-prefill buffers of this layer: raw fp16 slots for
        positions 0..capacity-1, the prefix length (device int32 [1]; 1 until a
        prefill is deferred, the reference's seed, :688-711) and the block-table
        row of the buffer."""
        pf = getattr(layer, "_fused_tq_prefix", None)
        if pf is None or pf[0].device != torch.device(device):
            nblk = (self._prefix_capacity + 15) // 16
            cache = torch.zeros(nblk, 16, self.num_kv_heads, RAW.raw_slot_bytes(self.head_size),
                                dtype=torch.uint8, device=device)
            plen = torch.ones(1, dtype=torch.int32, device=device)
            row = torch.arange(nblk, dtype=torch.int32, device=device)
            pf = (cache, plen, row)
            layer._fused_tq_prefix = pf
        return pf

    # -- store ---------------------------------------------------------------
    def do_kv_cache_update(self, layer, key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                           slot_mapping: torch.Tensor) -> None:
        N = slot_mapping.shape[0]
        if N <= 0:
            return
        if kv_cache.dtype != torch.uint8:
            kv_cache = kv_cache.view(torch.uint8)
        k = key[:N].reshape(N, self.num_kv_heads, self.head_size)
        v = value[:N].reshape(N, self.num_kv_heads, self.head_size)
        if self._is_raw:
            RAW.raw_store(k, v, kv_cache, slot_mapping[:N].to(torch.int64))
            return
        if self.defer_prefill and 1 < N <= self._prefix_capacity:
            # deferred prefill: fp16 copy at positions 0..N-1 of the prefix, no
            # quantised store (one sequence at a time, as in the reference)
            cache, plen, _ = self._prefix(layer, key.device)
            RAW.raw_store(k, v, cache, torch.arange(N, dtype=torch.int64, device=key.device))
            plen.fill_(N)
            return
        st = self._state(layer, key.device)
        st.store(k, v, kv_cache, slot_mapping[:N].to(torch.int64))

    # -- attention -----------------------------------------------------------
    def forward(self, layer, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                kv_cache: torch.Tensor, attn_metadata, output: Optional[torch.Tensor] = None,
                output_scale: Optional[torch.Tensor] = None,
                output_block_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
        num_tokens = query.shape[0]
        if output is None:
            output = torch.zeros(num_tokens, self.num_heads * self.head_size, dtype=query.dtype,
                                 device=query.device)
        if attn_metadata is None or attn_metadata.num_actual_tokens <= 0:
            return output.fill_(0)
        if kv_cache.dtype != torch.uint8:
            kv_cache = kv_cache.view(torch.uint8)
        N = attn_metadata.num_actual_tokens
        st = None if self._is_raw else self._state(layer, query.device)
        q = query[:N].view(N, self.num_heads, self.head_size)
        nd = attn_metadata.num_decodes
        ndt = attn_metadata.num_decode_tokens
        if not attn_metadata.is_prefill:
            nd, ndt = attn_metadata.seq_lens.shape[0], N
            # decode-only step: straight into vLLM's output buffer, per-layer
            # scratch, no host reads -- capturable in a CUDA/HIP graph
            o3 = output[:N].view(N, self.num_heads, self.head_size)
            if output.dtype == query.dtype and o3.is_contiguous():
                dec = self._decode_hybrid if self.defer_prefill else self._decode
                dec(q, kv_cache, attn_metadata.block_table[:nd], attn_metadata.seq_lens[:nd], st,
                    max_seq_len=getattr(attn_metadata, "max_seq_len", None), layer=layer, out=o3)
                return output
        out = torch.empty(N, self.num_heads, self.head_size, dtype=query.dtype, device=query.device)
        if ndt > 0:
            dec = self._decode_hybrid if self.defer_prefill else self._decode
            out[:ndt] = dec(q[:ndt], kv_cache, attn_metadata.block_table[:nd], attn_metadata.seq_lens[:nd], st,
                            max_seq_len=getattr(attn_metadata, "max_seq_len", None), layer=layer)
        if ndt < N:
            k = key[:N].view(N, self.num_kv_heads, self.head_size)
            v = value[:N].view(N, self.num_kv_heads, self.head_size)
            out[ndt:] = self._prefill(q, k, v, kv_cache, attn_metadata, nd, ndt, st)
        if output.ndim == 3:
            output[:N] = out.to(output.dtype)
        else:
            output[:N] = out.reshape(N, -1).to(output.dtype)
        return output

    def _splits(self, B: int, max_seq_len: int) -> int:
        """The decode's split-K factor: fixed (max_kv_splits) while a graph is
        being captured, else sized to the step's context, capped by it."""
        if torch.cuda.is_current_stream_capturing():
            return self.max_kv_splits
        if self._is_raw:
            s = RAW.default_splits(B, self.num_kv_heads, max_seq_len)
        else:
            flags = V1._v_flags(self.v_rotate, self.v_lloyd_max, self.key_fp8)
            s = V1.default_splits(B, self.num_kv_heads, max_seq_len, self.num_heads, self.head_size,
                                  self.key_bits, self.value_bits, flags)
        return max(1, min(self.max_kv_splits, s))

    def _decode_hybrid(self, q, kv_cache, block_table, seq_lens, st, max_seq_len=None, layer=None, out=None):
        """Deferred-prefill decode (reference _decode_attention_hybrid,
        :1095-1277): fp16 prefix attention for sequence 0, quantised attention
        over [P, seq_len) for every sequence, merged by log-sum-exp.  Every
        intermediate is per-layer scratch (no allocation after warm-up)."""
        B, hq, d = q.shape
        dev = q.device
        pcache, plen, row = self._prefix(layer, dev)
        bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
        sl = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
        msl = max_seq_len if max_seq_len is not None else bt.shape[1] * kv_cache.shape[1]
        # phase 1: the prefix, sequence 0 only (the others get no positions)
        sl_p = _buf(layer, "sl_p", (B,), torch.int32, dev)
        sl_p.zero_()
        sl_p[:1].copy_(plen)
        rows = _buf(layer, "prefix_rows", (B, row.shape[0]), torch.int32, dev)
        rows.copy_(row.expand(B, -1))
        o1 = _buf(layer, "o1", (B, hq, d), torch.float32, dev)
        l1 = _buf(layer, "l1", (B, hq), torch.float32, dev)
        s1 = RAW.default_splits(B, self.num_kv_heads, self._prefix_capacity)
        ws1 = _buf(layer, "ws1", (RAW.workspace_bytes(B, hq, d, s1),), torch.uint8, dev)
        RAW.raw_decode_attention(q, pcache, rows, sl_p, scale=self.scale, num_splits=s1, out=o1, lse=l1,
                                 workspace=ws1)
        # phase 2: the quantised positions [P, seq_len)
        o2 = _buf(layer, "o2", (B, hq, d), torch.float32, dev)
        l2 = _buf(layer, "l2", (B, hq), torch.float32, dev)
        ks = _buf(layer, "kv_start", (B,), torch.int32, dev)
        ks.copy_(plen.expand(B))
        s2 = self._splits(B, msl)
        ws2 = _buf(layer, "ws", (V1.workspace_bytes(B, hq, d, self.max_kv_splits),), torch.uint8, dev)
        V1.v1_decode_attention(q, kv_cache, bt, sl, st.centroids, self.key_bits, self.value_bits,
                               scale=self.scale, v_rotate=self.v_rotate, v_lloyd_max=self.v_lloyd_max,
                               kv_start=ks, num_splits=s2, out=o2, lse=l2, rotation=st.rotation,
                               workspace=ws2, sorted_centroids=True, key_fp8=self.key_fp8)
        # merge (a row empty in both phases stays 0)
        m = torch.maximum(l1, l2)
        m = torch.where(torch.isneginf(m), torch.zeros_like(m), m)
        w1, w2 = torch.exp(l1 - m), torch.exp(l2 - m)
        tot = (w1 + w2).clamp(min=1e-20)
        res = (o1 * w1.unsqueeze(-1) + o2 * w2.unsqueeze(-1)) / tot.unsqueeze(-1)
        if out is None:
            return res.to(q.dtype)
        out.copy_(res)
        return out

    def _decode(self, q, kv_cache, block_table, seq_lens, st, max_seq_len=None, layer=None, out=None):
        B, hq, d = q.shape
        dev = q.device
        bt = block_table if block_table.dtype == torch.int32 else block_table.to(torch.int32)
        sl = seq_lens if seq_lens.dtype == torch.int32 else seq_lens.to(torch.int32)
        msl = max_seq_len if max_seq_len is not None else bt.shape[1] * kv_cache.shape[1]
        splits = self._splits(B, msl)
        if layer is not None:
            wsb = (RAW.workspace_bytes if self._is_raw else V1.workspace_bytes)(B, hq, d, self.max_kv_splits)
            ws = _buf(layer, "ws", (wsb,), torch.uint8, dev)
        else:
            ws = None
        ks = None
        if self.sliding_window is not None:
            # each row attends its last W positions: [max(0, seq_len - W), seq_len)
            ks = _buf(layer, "win_start", (B,), torch.int32, dev) if layer is not None else \
                torch.empty(B, dtype=torch.int32, device=dev)
            torch.sub(sl, self.sliding_window, out=ks)
            ks.clamp_(min=0)
        if self._is_raw:
            return RAW.raw_decode_attention(q, kv_cache, bt, sl, scale=self.scale, kv_start=ks, num_splits=splits,
                                            out=out, workspace=ws)
        return V1.v1_decode_attention(q, kv_cache, bt, sl, st.centroids, self.key_bits, self.value_bits,
                                      scale=self.scale, v_rotate=self.v_rotate, v_lloyd_max=self.v_lloyd_max,
                                      kv_start=ks, num_splits=splits, rotation=st.rotation, out=out, workspace=ws,
                                      sorted_centroids=True, key_fp8=self.key_fp8)

    def _prefill(self, q, k, v, kv_cache, md, nd, ndt, st):
        """Prefill sequences nd.. of the batch (tokens ndt..N).  A run of
        consecutive fresh sequences of one length is one batched SDPA over
        views of q / k / v (no copies, grouped K/V); a continuing sequence
        runs the decode kernel with one synthetic row per query token."""
        qsl = md.query_start_loc.tolist()
        sls = md.seq_lens.tolist()
        N = q.shape[0]
        out = torch.empty(N - ndt, self.num_heads, self.head_size, dtype=q.dtype, device=q.device)
        n = len(sls)
        i = nd
        while i < n:
            a, b = qsl[i], qsl[i + 1]
            n_q = b - a
            if n_q == 0:
                i += 1
                continue
            past = sls[i] - n_q
            if past <= 0:
                # fresh sequences: causal attention over the full-precision K/V of the chunk
                j = i + 1
                while (j < n and qsl[j + 1] - qsl[j] == n_q and sls[j] == n_q
                       and (j + 1 - i) * n_q <= _FRESH_BATCH_TOKENS):
                    j += 1
                g = j - i
                e = a + g * n_q
                qq = q[a:e].view(g, n_q, self.num_heads, self.head_size)
                kk = k[a:e].view(g, n_q, self.num_kv_heads, self.head_size)
                vv = v[a:e].view(g, n_q, self.num_kv_heads, self.head_size)
                out[a - ndt:e - ndt] = self._fresh_attention(qq, kk, vv).reshape(g * n_q, self.num_heads,
                                                                                   self.head_size)
                i = j
            else:
                # continuation: one synthetic decode per query token over the stored slots
                row = md.block_table[i:i + 1].to(torch.int32).expand(n_q, -1).contiguous()
                syn = torch.arange(past + 1, past + n_q + 1, device=q.device, dtype=torch.int32)
                out[a - ndt:b - ndt] = self._decode(q[a:b], kv_cache, row, syn, st, max_seq_len=sls[i])
                i += 1
        return out

    def _fresh_attention(self, q, k, v):
        """Causal attention of fresh sequences, q [G, L, Hq, D] and k / v
        [G, L, Hkv, D] (views of the step's tensors) -> [G, L, Hq, D]; with a
        sliding window, query blocks attend their window of keys only."""
        G, L = q.shape[0], q.shape[1]
        qt, kt, vt = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        W = self.sliding_window
        if W is None or W >= L:
            return _sdpa(qt, kt, vt, self.scale).transpose(1, 2)
        out = torch.empty_like(q)
        pos = torch.arange(L, device=q.device)
        for a in range(0, L, _WINDOW_QUERY_BLOCK):
            b = min(L, a + _WINDOW_QUERY_BLOCK)
            k0 = max(0, a - W + 1)
            qi, kj = pos[a:b, None], pos[None, k0:b]
            mask = (kj <= qi) & (kj > qi - W)
            o = _sdpa(qt[:, :, a:b], kt[:, :, k0:b], vt[:, :, k0:b], self.scale, mask=mask)
            out[:, a:b] = o.transpose(1, 2)
        return out


# fresh prefill: tokens per batched SDPA launch, and query rows per block of a
# windowed one (its mask is block x (block + window) booleans)
_FRESH_BATCH_TOKENS = 32768
_WINDOW_QUERY_BLOCK = 2048
_GQA_KERNELS: Optional[bool] = None  # whether torch's fused SDPA kernels take grouped K/V here


def _sdpa(q, k, v, scale: float, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(q k^T * scale) v over [G, H, L, D] views, causal (mask None)
    or under a boolean mask.  Causal grouped K/V (Hkv < Hq) go to torch's
    fused kernels with ``enable_gqa`` (the reference's call,
    v1_backend.py:1355-1358); where those kernels refuse grouped heads, and
    under a mask (torch's flash kernel takes no mask and its memory-efficient
    one no grouped heads), K/V are expanded once per call."""
    global _GQA_KERNELS
    from torch.nn.attention import SDPBackend, sdpa_kernel
    rep = q.shape[1] // k.shape[1]
    kw = dict(attn_mask=mask, is_causal=mask is None, scale=scale)
    if rep > 1 and mask is None and _GQA_KERNELS is not False:
        try:
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                o = F.scaled_dot_product_attention(q, k, v, enable_gqa=True, **kw)
            _GQA_KERNELS = True
            return o
        except RuntimeError:
            _GQA_KERNELS = False
    if rep > 1:
        k = k.repeat_interleave(rep, dim=1)
        v = v.repeat_interleave(rep, dim=1)
    return F.scaled_dot_product_attention(q, k, v, **kw)
