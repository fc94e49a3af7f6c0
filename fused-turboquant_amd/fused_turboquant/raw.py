"""Raw fp16 KV slots of the vLLM ``TURBOQUANT`` backend's boundary layers on
gfx950: store and split-K decode attention.

With ``TURBOQUANT_BOUNDARY_PROTECT=fp16`` (the reference's default) vLLM keeps
the first and last attention layers unquantised, in the same byte allocation
as the TurboQuant layers, ``uint8[num_blocks, block_size, num_kv_heads, slot]``;
one slot holds, per (token, kv head), ``[K fp16 (2 d B)][V fp16 (2 d B)][pad]``
(reference ``vllm_plugin/v1_backend.py:1449-1505``).

* ``raw_store`` replaces ``_store_raw_kv`` (``v1_backend.py:1449-1505``):
  K and V rounded to fp16, negative slots skipped.
* ``raw_decode_attention`` replaces ``boundary_fp16_decode_attention``
  (``vllm_plugin/triton_boundary_attn.py:28-219``) as called by
  ``_forward_raw`` (``v1_backend.py:1547-1640``).
"""
from __future__ import annotations

import math

import torch

from . import _lib, _ops

_SIG = {
    "ftq_raw_store": ["vp", "vp", "i32", "i64", "i32", "i32", "vp", "vp", "i64", "i32", "i64", "i64",
                      "i64", "vp"],
    "ftq_raw_decode_attention": ["vp", "i32", "vp", "i64", "i32", "i64", "i64", "i64", "vp", "i32",
                                 "vp", "vp", "i32", "i32", "i32", "i32", "f32", "i32", "vp", "i64",
                                 "vp", "i32", "vp"],
    "ftq_raw_decode_attention_lse": ["vp", "i32", "vp", "i64", "i32", "i64", "i64", "i64", "vp", "i32",
                                     "vp", "vp", "i32", "i32", "i32", "i32", "f32", "i32", "vp", "i64",
                                     "vp", "i32", "vp", "vp"],
}


def _bind():
    import ctypes
    L = _lib.lib()
    if getattr(L, "_raw_bound", False):
        return L
    m = {"vp": ctypes.c_void_p, "i32": ctypes.c_int, "i64": ctypes.c_int64, "f32": ctypes.c_float}
    for name, sig in _SIG.items():
        fn = getattr(L, name)
        fn.argtypes = [m[t] for t in sig]
        fn.restype = ctypes.c_int
    L.ftq_raw_slot_bytes.restype = ctypes.c_int64
    L.ftq_raw_slot_bytes.argtypes = [ctypes.c_int]
    L.ftq_raw_workspace_bytes.restype = ctypes.c_int64
    L.ftq_raw_workspace_bytes.argtypes = [ctypes.c_int] * 4
    L.ftq_raw_default_splits.restype = ctypes.c_int
    L.ftq_raw_default_splits.argtypes = [ctypes.c_int] * 3
    L._raw_bound = True
    return L


def raw_slot_bytes(head_dim: int) -> int:
    """Bytes of a raw slot that hold data: K and V in fp16."""
    if head_dim not in (64, 128, 256):
        raise ValueError(f"head_dim must be 64, 128 or 256, got {head_dim}")
    return 4 * head_dim


def _strides(kv_cache: torch.Tensor):
    if kv_cache.dtype != torch.uint8 or kv_cache.dim() != 4:
        raise ValueError("kv_cache must be uint8 [num_blocks, block_size, num_kv_heads, slot]")
    if kv_cache.stride(3) != 1:
        raise ValueError("kv_cache slot bytes must be contiguous")
    return kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2)


def raw_store(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
    """Write ``key``/``value`` [n, Hkv, d] as fp16 into their raw slots
    (``slot_mapping`` [n] int64; negative entries are skipped)."""
    n, hkv, d = key.shape
    if value.shape != key.shape:
        raise ValueError("key and value shapes differ")
    nb, bs, hk2, slot = kv_cache.shape
    if hk2 != hkv:
        raise ValueError("kv_cache num_kv_heads does not match key")
    if slot < raw_slot_bytes(d):
        raise ValueError("kv_cache slot is smaller than 4 * head_dim bytes")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != n:
        raise ValueError("slot_mapping must be int64 with one entry per token")
    dev = _lib.require_device(key, value, kv_cache, slot_mapping)
    k = key.contiguous()
    if k.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        k = k.float()
    v = value.to(k.dtype).contiguous()
    _strides(kv_cache)
    del dev
    _ops.ops().raw_store(k, v, kv_cache, slot_mapping.contiguous())


def default_splits(batch: int, num_kv_heads: int, max_seq_len: int) -> int:
    return int(_bind().ftq_raw_default_splits(batch, num_kv_heads, max_seq_len))


def workspace_bytes(batch: int, num_q_heads: int, head_dim: int, num_splits: int) -> int:
    return int(_bind().ftq_raw_workspace_bytes(batch, num_q_heads, head_dim, num_splits))


def raw_decode_attention(query: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                         seq_lens: torch.Tensor, scale: float | None = None,
                         kv_start: torch.Tensor | None = None, num_splits: int | None = None,
                         max_seq_len: int | None = None, out: torch.Tensor | None = None,
                         workspace: torch.Tensor | None = None, lse: torch.Tensor | None = None) -> torch.Tensor:
    """query [B, Hq, d] -> [B, Hq, d] (query dtype unless ``out`` is given).

    Attends positions [kv_start[b], seq_lens[b]) of block-table row b over the
    raw fp16 slots.  Head dim 128 runs the matrix-core kernel (GQA group <= 8);
    64 and 256 the fp32 VALU kernel (group <= 16).  ``num_splits`` defaults to a value that fills the GPU
    (pass ``max_seq_len`` to size it without reading ``block_table``'s width);
    ``workspace`` (uint8, >= ``workspace_bytes``) may be preallocated.
    ``lse`` (float32 [B, Hq]) receives each row's natural-log log-sum-exp of
    the scaled scores (-inf for a row with no positions).
    """
    B, hq, d = query.shape
    nb, bs, hkv, slot = kv_cache.shape
    if slot < raw_slot_bytes(d):
        raise ValueError("kv_cache slot is smaller than 4 * head_dim bytes")
    gmax = 8 if d == 128 else 16
    if hq % hkv != 0 or hq // hkv > gmax:
        raise ValueError(f"num_q_heads must be a multiple of num_kv_heads with a group of at most {gmax}")
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("block_table and seq_lens must be int32")
    if block_table.dim() != 2 or block_table.shape[0] != B or seq_lens.numel() != B:
        raise ValueError("block_table must be [B, max_blocks] and seq_lens [B]")
    if kv_start is not None and (kv_start.dtype != torch.int32 or kv_start.numel() != B):
        raise ValueError("kv_start must be int32 [B]")
    if lse is not None and (lse.dtype != torch.float32 or lse.numel() != B * hq or not lse.is_contiguous()):
        raise ValueError("lse must be a contiguous float32 tensor of B * num_q_heads entries")
    tensors = [query, kv_cache, block_table, seq_lens] + ([kv_start] if kv_start is not None else [])
    tensors += [lse] if lse is not None else []
    dev = _lib.require_device(*tensors)
    q = query.contiguous()
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        q = q.float()
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if num_splits is None:
        msl = max_seq_len if max_seq_len is not None else block_table.shape[1] * bs
        num_splits = default_splits(B, hkv, msl)
    if out is None:
        out = torch.empty(B, hq, d, dtype=q.dtype, device=dev)
    need = workspace_bytes(B, hq, d, num_splits)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    _strides(kv_cache)
    ks = kv_start.contiguous() if kv_start is not None else None
    _ops.ops().raw_decode_attention(q, kv_cache, block_table.contiguous(), seq_lens.contiguous(), ks,
                                    float(scale), int(num_splits), workspace, out, lse)
    return out
