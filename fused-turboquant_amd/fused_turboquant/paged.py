"""Paged TurboQuant KV cache (library format) with fused decode attention on gfx950.

The library format is the one ``TurboQuantMSE`` produces (RHT with random
signs, Lloyd-Max codebook, fp16 norm of the rotated vector; reference
``core/quantizer.py:137-160``).  This module keeps it in pages addressed by a
block table, as a vLLM-style paged backend does, and computes decode
attention straight from the packed codes:

* ``paged_store`` -- encode K and V of new tokens and scatter them to their
  slots (``slot = block * page_size + offset``; negative slots are skipped,
  like the reference store, ``vllm_plugin/triton_inkernel_store.py:398-399``).
* ``paged_decode_attention`` -- one query token per sequence; semantics of the
  reference's library-format decode (``vllm_plugin/attention_impl.py:431-521``,
  ``kernels/triton_flash_decode.py:66-221``): softmax(q . K^T * scale) . V over
  the decoded cache, GQA head h -> kv head h // (Hq / Hkv), positions
  >= seq_lens[b] masked.

Cache layout: ``uint8[num_blocks, num_kv_heads, page_size // 16, sub_bytes]``
(see ``csrc/ftq_paged.hip`` for the byte layout of one 16-token sub-block).
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib, _ops
from .core.quantizer import TurboQuantMSE

_SIG = {
    "ftq_paged_store": ["vp", "vp", "i32", "i64", "i32", "i32", "vp", "vp", "vp", "vp", "i32", "i32",
                        "vp", "vp", "i32", "i64", "vp"],
    "ftq_paged_decode_attention": ["vp", "i32", "vp", "vp", "vp", "i32", "i32", "i32", "i32", "i32",
                                   "i32", "i64", "vp", "vp", "vp", "vp", "i32", "i32", "f32", "i32",
                                   "vp", "i64", "vp", "i32", "vp"],
}
_SIG["ftq_paged_decode_attention_valu"] = _SIG["ftq_paged_decode_attention"]


def _bind():
    import ctypes
    L = _lib.lib()
    if getattr(L, "_paged_bound", False):
        return L
    m = {"vp": ctypes.c_void_p, "i32": ctypes.c_int, "i64": ctypes.c_int64, "f32": ctypes.c_float}
    for name, sig in _SIG.items():
        fn = getattr(L, name)
        fn.argtypes = [m[t] for t in sig]
        fn.restype = ctypes.c_int
    for name in ("ftq_paged_subblock_bytes",):
        getattr(L, name).restype = ctypes.c_int64
        getattr(L, name).argtypes = [ctypes.c_int] * 3
    L.ftq_paged_workspace_bytes.restype = ctypes.c_int64
    L.ftq_paged_workspace_bytes.argtypes = [ctypes.c_int] * 4
    L.ftq_paged_default_splits.restype = ctypes.c_int
    L.ftq_paged_default_splits.argtypes = [ctypes.c_int] * 3
    L.ftq_paged_choose_splits.restype = ctypes.c_int
    L.ftq_paged_choose_splits.argtypes = [ctypes.c_int] * 5
    L._paged_bound = True
    return L


def subblock_bytes(head_dim: int, bits_k: int, bits_v: int) -> int:
    """Bytes of one 16-token sub-block of one kv head: 2*d*(bk+bv) + 64."""
    if head_dim not in (128, 256) or not (2 <= bits_k <= 4) or not (2 <= bits_v <= 4):
        raise ValueError("paged cache supports head_dim 128/256 and 2/3/4-bit K and V")
    return 2 * head_dim * (bits_k + bits_v) + 64


def cache_shape(num_blocks: int, page_size: int, num_kv_heads: int, head_dim: int,
                bits_k: int, bits_v: int) -> tuple:
    if page_size % 16 != 0 or page_size <= 0:
        raise ValueError("page_size must be a positive multiple of 16")
    return (num_blocks, num_kv_heads, page_size // 16, subblock_bytes(head_dim, bits_k, bits_v))


def paged_store(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
                slot_mapping: torch.Tensor, k_quant: TurboQuantMSE, v_quant: TurboQuantMSE) -> None:
    """Encode ``key``/``value`` [n, Hkv, d] and write them to ``slot_mapping`` [n] (int64)."""
    n, hkv, d = key.shape
    if value.shape != key.shape:
        raise ValueError("key and value shapes differ")
    nb, hk2, nsub, sub = kv_cache.shape
    if hk2 != hkv or sub != subblock_bytes(d, k_quant.bits, v_quant.bits) or kv_cache.dtype != torch.uint8:
        raise ValueError("kv_cache shape does not match (num_kv_heads, head_dim, bits)")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != n:
        raise ValueError("slot_mapping must be int64 with one entry per token")
    dev = _lib.require_device(key, value, kv_cache, slot_mapping)
    k = key.contiguous()
    v = value.to(k.dtype).contiguous()
    if k.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        k, v = k.float(), v.float()
    del dev
    _ops.ops().paged_store(k, v, kv_cache, slot_mapping.contiguous(), k_quant.rotation.signs,
                           v_quant.rotation.signs, k_quant.quantizer.boundaries, v_quant.quantizer.boundaries,
                           k_quant.bits, v_quant.bits, nsub * 16)


def default_splits(batch: int, num_kv_heads: int, max_seq_len: int, num_q_heads: int | None = None,
                   head_dim: int | None = None) -> int:
    """Split factor of the decode: with ``num_q_heads`` and ``head_dim`` it may
    be 1, the single-launch form (d = 128, GQA group <= 4, batch * Hkv filling
    the GPU); without them, the split form's own default."""
    if num_q_heads is not None and head_dim is not None:
        return int(_bind().ftq_paged_choose_splits(batch, num_q_heads, num_kv_heads, head_dim, max_seq_len))
    return int(_bind().ftq_paged_default_splits(batch, num_kv_heads, max_seq_len))


def _levels_pair(k_quant: TurboQuantMSE, v_quant: TurboQuantMSE):
    """Device pointers of the K and V levels; one pointer for both when the two
    codebooks are equal (the kernel then builds one shared code table)."""
    kq, vq = k_quant.quantizer, v_quant.quantizer
    if kq is vq or (kq.bits == vq.bits and np.array_equal(kq.levels_host, vq.levels_host)):
        return kq.levels.data_ptr(), kq.levels.data_ptr()
    return kq.levels.data_ptr(), vq.levels.data_ptr()


def _levels_tensors(k_quant: TurboQuantMSE, v_quant: TurboQuantMSE):
    """The K and V level tensors; the K tensor for both when the codebooks are
    equal (the kernel then builds one shared code table)."""
    kp, vp = _levels_pair(k_quant, v_quant)
    kl = k_quant.quantizer.levels
    return kl, (kl if kp == vp else v_quant.quantizer.levels)


def workspace_bytes(batch: int, num_q_heads: int, head_dim: int, num_splits: int) -> int:
    return int(_bind().ftq_paged_workspace_bytes(batch, num_q_heads, head_dim, num_splits))


def paged_decode_attention(query: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                           seq_lens: torch.Tensor, k_quant: TurboQuantMSE, v_quant: TurboQuantMSE,
                           scale: float | None = None, num_splits: int | None = None,
                           max_seq_len: int | None = None, out: torch.Tensor | None = None,
                           workspace: torch.Tensor | None = None, operands: str = "f16") -> torch.Tensor:
    """query [B, Hq, d] -> attention output [B, Hq, d] (query dtype unless ``out`` given).

    ``num_splits`` (split-K factor over the context) defaults to a value that
    fills the GPU; pass ``max_seq_len`` to size it without a device sync.
    ``workspace`` (uint8, >= ``workspace_bytes``) may be preallocated for
    graph capture.  ``operands``: ``"f16"`` (default) takes the scores and
    P.V on the matrix cores with f16 operands (scaled level tables, query as
    f16 hi + lo, fp32 accumulation); ``"fp32"`` takes every product in fp32
    on the VALU, the reference's arithmetic (d = 128, GQA group <= 4, split
    form only).
    """
    if operands not in ("f16", "fp32"):
        raise ValueError("operands must be 'f16' or 'fp32'")
    B, hq, d = query.shape
    nb, hkv, nsub, sub = kv_cache.shape
    if sub != subblock_bytes(d, k_quant.bits, v_quant.bits):
        raise ValueError("kv_cache sub-block size does not match (head_dim, bits)")
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("block_table and seq_lens must be int32")
    if block_table.dim() != 2 or block_table.shape[0] != B or seq_lens.numel() != B:
        raise ValueError("block_table must be [B, max_blocks] and seq_lens [B]")
    dev = _lib.require_device(query, kv_cache, block_table, seq_lens)
    q = query.contiguous()
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        q = q.float()
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if num_splits is None:
        msl = max_seq_len if max_seq_len is not None else block_table.shape[1] * nsub * 16
        num_splits = default_splits(B, hkv, msl, hq, d) if operands == "f16" else default_splits(B, hkv, msl)
    if out is None:
        out = torch.empty(B, hq, d, dtype=q.dtype, device=dev)
    need = workspace_bytes(B, hq, d, num_splits)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    bt = block_table.contiguous()
    if operands == "fp32" and (d != 128 or hq // hkv > 4):
        raise ValueError("fp32 operands: head_dim 128 and at most 4 query heads per kv head")
    _ops.ops().paged_decode_attention(
        q, kv_cache, bt, seq_lens.contiguous(), k_quant.rotation.signs, v_quant.rotation.signs,
        *_levels_tensors(k_quant, v_quant), k_quant.bits, v_quant.bits, nsub * 16, float(scale),
        int(num_splits), workspace, out, operands == "fp32")
    return out


_V_GATHER: dict = {}


def _v_gather_index(head_dim: int, bits_v: int, device) -> torch.Tensor:
    """Bit index, into the 64 V lane chunks of a sub-block laid out as one bit
    stream, of bit k of the code of (token t, dim e): chunk 16 (t // 4) + e % 16,
    bit (4 (e // 16) + t % 4) bits_v + k.  Shape [16, head_dim, bits_v]."""
    key = (head_dim, bits_v, str(device))
    if key not in _V_GATHER:
        vlane_bits = head_dim * bits_v // 4
        t = torch.arange(16).view(16, 1, 1)
        e = torch.arange(head_dim).view(1, head_dim, 1)
        k = torch.arange(bits_v).view(1, 1, bits_v)
        chunk = 16 * (t // 4) + e % 16
        bit = (4 * (e // 16) + t % 4) * bits_v + k
        _V_GATHER[key] = (chunk * vlane_bits + bit).to(device)
    return _V_GATHER[key]


def _pack_codes(codes: torch.Tensor, bits: int) -> torch.Tensor:
    from .core.packing import pack_2bit, pack_3bit, pack_nibbles
    return {2: pack_2bit, 3: pack_3bit, 4: pack_nibbles}[bits](codes)


def paged_read(kv_cache: torch.Tensor, blocks: torch.Tensor, head_dim: int, bits_k: int,
               bits_v: int):
    """Codes and norms of the pages ``blocks`` [n] in the flat library format
    (``CompressedTensor`` layout, reference ``core/packing.py``):
    K packed [n, Hkv, page, d*bk/8], K norms [n, Hkv, page] f16, and the same
    for V.  Plain torch gathers on the device (not on the decode path: the
    attention kernel reads pages directly)."""
    nb, hkv, nsub, sub = kv_cache.shape
    ktok = head_dim * bits_k // 8
    ksec = 16 * ktok
    vsec = 64 * (head_dim * bits_v // 32)
    if sub != ksec + vsec + 64:
        raise ValueError("kv_cache sub-block size does not match (head_dim, bits)")
    c = kv_cache.index_select(0, blocks.to(torch.int64))  # [n, Hkv, nsub, sub]
    n = c.shape[0]
    k_packed = c[..., :ksec].reshape(n, hkv, nsub * 16, ktok)
    norms = c[..., ksec + vsec:].contiguous().view(torch.float16)  # [n, Hkv, nsub, 32]
    k_norms = norms[..., :16].reshape(n, hkv, nsub * 16)
    v_norms = norms[..., 16:].reshape(n, hkv, nsub * 16)
    vbytes = c[..., ksec:ksec + vsec].to(torch.int32)  # [n, Hkv, nsub, vsec]
    vbits = ((vbytes.unsqueeze(-1) >> torch.arange(8, device=c.device, dtype=torch.int32)) & 1)
    vbits = vbits.reshape(n, hkv, nsub, vsec * 8)
    idx = _v_gather_index(head_dim, bits_v, c.device)
    g = vbits[..., idx.reshape(-1)].reshape(n, hkv, nsub, 16, head_dim, bits_v)
    v_codes = (g << torch.arange(bits_v, device=c.device, dtype=torch.int32)).sum(-1)
    v_packed = _pack_codes(v_codes.reshape(n, hkv, nsub * 16, head_dim), bits_v)
    return k_packed, k_norms, v_packed, v_norms


class PagedTurboQuantCache:
    """A paged, compressed KV cache of one attention layer.

    K and V get their own ``TurboQuantMSE`` (same seed by default, as
    ``patch_model`` shares one quantizer per (head_dim, bits) across K and V,
    reference ``hf/fused_cache.py:1143-1202``).
    """

    def __init__(self, num_blocks: int, page_size: int, num_kv_heads: int, head_dim: int,
                 bits_k: int = 3, bits_v: int = 3, seed: int = 42, device="cuda"):
        self.page_size = page_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.k_quant = TurboQuantMSE(head_dim, bits=bits_k, seed=seed, device=device)
        self.v_quant = TurboQuantMSE(head_dim, bits=bits_v, seed=seed, device=device)
        self.kv_cache = torch.zeros(cache_shape(num_blocks, page_size, num_kv_heads, head_dim, bits_k, bits_v),
                                    dtype=torch.uint8, device=device)

    def store(self, key: torch.Tensor, value: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        paged_store(key, value, self.kv_cache, slot_mapping, self.k_quant, self.v_quant)

    def decode_attention(self, query, block_table, seq_lens, **kw) -> torch.Tensor:
        return paged_decode_attention(query, self.kv_cache, block_table, seq_lens,
                                      self.k_quant, self.v_quant, **kw)
