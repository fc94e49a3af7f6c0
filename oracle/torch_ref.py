"""Torch restatement of the reference's unfused CPU path, used as the CPU
baseline that ``bench.py`` times (and pinned by ``tests/test_oracle.py``
against the reference's golden fixtures and the numpy oracle).

TEST / MEASUREMENT INFRASTRUCTURE ONLY: nothing in the product package imports
this module.  It restates, in torch on the host:

* ``rht`` / ``inverse_rht``: ``core/hadamard.py:23-48`` (``fwht``: log2 d
  stages of (a + b, a - b) over halves of stride h = 1, 2, 4, ..., then times
  the float32 constant d**-0.5) and ``:70-100`` (``fwht(x * signs)``,
  ``fwht(y) * signs``).
* ``encode``: ``TurboQuantMSE._encode_unfused`` (``core/quantizer.py:137-160``):
  x.float(), rotate, ``torch.norm`` over the last dim,
  ``rotated / (norm + 1e-8)``, ``bucketize(u, boundaries) - 1`` clamped
  (``core/lloyd_max.py:121-132``), pack (``core/packing.py:14-128``), norms
  to fp16.
* ``decode``: ``_decode_unfused`` (``core/quantizer.py:191-205``): unpack,
  ``levels[idx] * norm``, inverse RHT; float32 out.
* ``dense_attention``: decode attention over decoded K / V (scores, softmax,
  weighted sum) in float32, the semantics of ``attention_impl.py:431-521``.
"""
from __future__ import annotations

import torch


def fwht(x: torch.Tensor) -> torch.Tensor:
    """Orthonormal Walsh-Hadamard transform over the last dim (core/hadamard.py:23-48)."""
    d = x.shape[-1]
    lead = x.shape[:-1]
    h = 1
    while h < d:
        v = x.reshape(*lead, d // (2 * h), 2, h)
        a, b = v.unbind(-2)
        x = torch.stack((a + b, a - b), dim=-2).reshape(*lead, d)
        h *= 2
    return x * (d ** -0.5)


def rht(x: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    return fwht(x * signs)


def inverse_rht(y: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    return fwht(y) * signs


def pack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Codes [..., d] (uint8) -> bytes [..., d * bits / 8]: each group of
    codes (2 per byte at 4 bits, 4 per byte at 2 bits, 8 per 3 bytes at 3
    bits) forms an integer with code k of the group at bit k * bits, written
    out little-endian (core/packing.py:14-128)."""
    d = codes.shape[-1]
    per = {2: 4, 3: 8, 4: 2}[bits]
    nbytes = per * bits // 8
    c = codes.reshape(*codes.shape[:-1], d // per, per).to(torch.int64)
    word = (c << (bits * torch.arange(per, dtype=torch.int64))).sum(-1)
    out = (word[..., None] >> (8 * torch.arange(nbytes, dtype=torch.int64))) & 0xFF
    return out.to(torch.uint8).reshape(*codes.shape[:-1], d * bits // 8)


def unpack(packed: torch.Tensor, bits: int, d: int) -> torch.Tensor:
    per = {2: 4, 3: 8, 4: 2}[bits]
    nbytes = per * bits // 8
    b = packed.reshape(*packed.shape[:-1], d // per, nbytes).to(torch.int64)
    word = (b << (8 * torch.arange(nbytes, dtype=torch.int64))).sum(-1)
    c = (word[..., None] >> (bits * torch.arange(per, dtype=torch.int64))) & ((1 << bits) - 1)
    return c.to(torch.uint8).reshape(*packed.shape[:-1], d)


def encode(x: torch.Tensor, signs: torch.Tensor, boundaries: torch.Tensor, bits: int):
    """-> (packed uint8 [..., d*bits/8], norms float16 [...])."""
    y = rht(x.float(), signs)
    norms = torch.norm(y, dim=-1, keepdim=True)
    u = y / (norms + 1e-8)
    idx = (torch.bucketize(u, boundaries) - 1).clamp(0, (1 << bits) - 1).to(torch.uint8)
    return pack(idx, bits), norms.squeeze(-1).half()


def decode(packed: torch.Tensor, norms: torch.Tensor, levels: torch.Tensor, signs: torch.Tensor,
           bits: int, d: int) -> torch.Tensor:
    idx = unpack(packed, bits, d)
    rec = levels[idx.long()] * norms.float().unsqueeze(-1)
    return inverse_rht(rec, signs)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """q [B, Hq, d], k / v [B, Hkv, S, d] (float32) -> [B, Hq, d]; query head h
    reads kv head h // (Hq / Hkv)."""
    B, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    qg = q.float().reshape(B, hkv, g, d)
    s = torch.matmul(qg, k.transpose(-1, -2)) * scale          # [B, Hkv, G, S]
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v).reshape(B, hq, d)
