"""Sub-byte packing layouts (reference ``core/packing.py:14-128``).

The fused kernels pack and unpack in registers; these torch helpers exist for
callers of the reference API that pack indices themselves.  Layouts:
4-bit low nibble = even index; 2-bit four codes per byte, LSB first; 3-bit
eight codes -> 24-bit little-endian word in 3 bytes, code k at bits 3k..3k+2.
"""
from __future__ import annotations

import torch


def pack_nibbles(indices: torch.Tensor) -> torch.Tensor:
    assert indices.shape[-1] % 2 == 0, "Last dimension must be even for nibble packing"
    v = indices.reshape(*indices.shape[:-1], -1, 2).to(torch.uint8)
    return (v[..., 1] << 4) | v[..., 0]


def unpack_nibbles(packed: torch.Tensor, original_dim: int) -> torch.Tensor:
    return torch.stack([packed & 0x0F, (packed >> 4) & 0x0F], dim=-1).reshape(
        *packed.shape[:-1], original_dim)


def pack_2bit(indices: torch.Tensor) -> torch.Tensor:
    assert indices.shape[-1] % 4 == 0, "Last dimension must be divisible by 4 for 2-bit packing"
    v = indices.reshape(*indices.shape[:-1], -1, 4).to(torch.uint8)
    return v[..., 0] | (v[..., 1] << 2) | (v[..., 2] << 4) | (v[..., 3] << 6)


def unpack_2bit(packed: torch.Tensor, original_dim: int) -> torch.Tensor:
    return torch.stack([(packed >> s) & 0x03 for s in (0, 2, 4, 6)], dim=-1).reshape(
        *packed.shape[:-1], original_dim)


def pack_3bit(indices: torch.Tensor) -> torch.Tensor:
    d = indices.shape[-1]
    assert d % 8 == 0, "Last dimension must be divisible by 8 for 3-bit packing"
    v = indices.reshape(*indices.shape[:-1], -1, 8).to(torch.int32) & 7
    w = torch.zeros(v.shape[:-1], dtype=torch.int32, device=v.device)
    for k in range(8):
        w = w | (v[..., k] << (3 * k))
    out = torch.stack([w & 255, (w >> 8) & 255, (w >> 16) & 255], dim=-1).to(torch.uint8)
    return out.reshape(*indices.shape[:-1], d * 3 // 8)


def unpack_3bit(packed: torch.Tensor, original_dim: int) -> torch.Tensor:
    g = packed.reshape(*packed.shape[:-1], -1, 3).to(torch.int32)
    w = g[..., 0] | (g[..., 1] << 8) | (g[..., 2] << 16)
    return torch.stack([(w >> (3 * k)) & 7 for k in range(8)], dim=-1).to(torch.uint8).reshape(
        *packed.shape[:-1], original_dim)
