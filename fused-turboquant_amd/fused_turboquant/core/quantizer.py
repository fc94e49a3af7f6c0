"""TurboQuant_MSE encode / decode on gfx950.

Mirrors reference ``core/quantizer.py``: ``CompressedTensor`` (:36-51) and
``TurboQuantMSE`` (:54-216).  ``encode`` and ``decode`` are single HIP kernel
launches (``ftq_encode`` / ``ftq_decode``) with the numerics of the
reference's unfused path (:137-160, :191-205): packed codes, fp16 norms of
the rotated vector, float32 reconstruction.  Device tensors only; the
launches go through the ``torch.ops.fused_tq.encode`` / ``decode`` operators.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .. import _lib, _ops
from .hadamard import RHTRotation
from .lloyd_max import LloydMaxQuantizer


def packed_dim(head_dim: int, bits: int) -> int:
    return head_dim * bits // 8


@dataclass
class CompressedTensor:
    """Compressed representation of a tensor after TurboQuant encoding."""

    indices: torch.Tensor  # packed uint8 quantization indices [..., d*bits/8]
    norms: torch.Tensor  # fp16 vector norms (1 per vector)
    original_dim: int
    bits: int

    @property
    def compression_ratio(self) -> float:
        original_bytes = self.norms.numel() * self.original_dim * 2
        compressed_bytes = self.indices.numel() + self.norms.numel() * 2
        if compressed_bytes == 0:
            return float("inf")
        return original_bytes / compressed_bytes


class TurboQuantMSE:
    """TurboQuant_MSE: RHT + Lloyd-Max encode/decode pipeline.

    Usage (reference quantizer.py:54-66):
        tq = TurboQuantMSE(head_dim=128, bits=3, device="cuda")
        ct = tq.encode(k)          # (..., head_dim) -> CompressedTensor
        k_hat = tq.decode(ct)      # CompressedTensor -> (..., head_dim) float32
    """

    def __init__(self, head_dim: int, bits: int = 4, seed: int = 42,
                 device: torch.device | str = "cpu", max_iterations: int = 300,
                 num_grid_points: int = 50000):
        if head_dim < 1 or (head_dim & (head_dim - 1)) != 0:
            raise ValueError(f"head_dim must be a power of 2, got {head_dim}")
        if bits not in (2, 3, 4):
            raise ValueError(f"bits must be 2, 3, or 4, got {bits}")
        if not 8 <= head_dim <= 4096:
            # 64 / 128 / 256 run tuned kernels; the other powers of two a generic one
            raise ValueError(f"head_dim must be a power of two in [8, 4096] for the gfx950 kernels, "
                             f"got {head_dim}")
        self.head_dim = head_dim
        self.bits = bits
        self.device = device
        self.rotation = RHTRotation(head_dim, seed=seed, device=device)
        self.quantizer = LloydMaxQuantizer(head_dim, bits=bits, device=device,
                                           max_iterations=max_iterations,
                                           num_grid_points=num_grid_points)

    # -- encode ------------------------------------------------------------
    def encode(self, x: torch.Tensor) -> CompressedTensor:
        if x.shape[-1] != self.head_dim:
            raise ValueError(f"last dim {x.shape[-1]} != head_dim {self.head_dim}")
        dev = _lib.require_device(x, self.rotation.signs, self.quantizer.boundaries)
        xc = x.contiguous()
        if xc.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            xc = xc.float()
        del dev
        packed, norms = _ops.ops().encode(xc, self.rotation.signs, self.quantizer.boundaries, self.bits,
                                          self.quantizer.codebook_class)
        return CompressedTensor(indices=packed, norms=norms, original_dim=self.head_dim, bits=self.bits)

    def encode_kv(self, k: torch.Tensor, v: torch.Tensor) -> tuple[CompressedTensor, CompressedTensor]:
        """``(encode(k), encode(v))`` of two tensors of one shape and dtype, in
        one kernel launch for 16-bit input at d = 128 / 256 -- the stacked
        K + V encode of ``FusedTurboQuantCache.store_compressed_kv``
        (reference ``hf/fused_cache.py:274-330``) without the stack copy."""
        if k.shape != v.shape or k.dtype != v.dtype:
            raise ValueError(f"k {tuple(k.shape)} {k.dtype} and v {tuple(v.shape)} {v.dtype} must agree")
        if k.shape[-1] != self.head_dim:
            raise ValueError(f"last dim {k.shape[-1]} != head_dim {self.head_dim}")
        _lib.require_device(k, v, self.rotation.signs, self.quantizer.boundaries)
        kc, vc = k.contiguous(), v.contiguous()
        if kc.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            kc, vc = kc.float(), vc.float()
        kp, kn, vp, vn = _ops.ops().encode_kv(kc, vc, self.rotation.signs, self.quantizer.boundaries, self.bits,
                                              self.quantizer.codebook_class)
        return (CompressedTensor(indices=kp, norms=kn, original_dim=self.head_dim, bits=self.bits),
                CompressedTensor(indices=vp, norms=vn, original_dim=self.head_dim, bits=self.bits))

    # -- decode ------------------------------------------------------------
    def decode(self, compressed: CompressedTensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        d, bits = compressed.original_dim, compressed.bits
        if d != self.head_dim:
            raise ValueError(f"original_dim {d} != head_dim {self.head_dim}")
        pk = compressed.indices.contiguous()
        nr = compressed.norms.contiguous()
        if pk.dtype != torch.uint8 or pk.shape[-1] != packed_dim(d, bits):
            raise ValueError("indices must be uint8 with last dim d*bits/8")
        if nr.dtype != torch.float16 or tuple(nr.shape) != tuple(pk.shape[:-1]):
            raise ValueError("norms must be float16 with the leading shape of indices")
        _lib.require_device(pk, nr, self.quantizer.levels)
        _lib.dtype_code(out_dtype)
        return _ops.ops().decode(pk, nr, self.quantizer.levels, self.rotation.signs, bits, d, out_dtype)

    def roundtrip(self, x: torch.Tensor) -> torch.Tensor:
        return self.decode(self.encode(x))

    def to(self, device: torch.device | str) -> "TurboQuantMSE":
        self.device = device
        self.rotation = self.rotation.to(device)
        self.quantizer = self.quantizer.to(device)
        return self
