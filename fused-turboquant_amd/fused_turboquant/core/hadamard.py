"""Randomized Hadamard Transform on gfx950.

Mirrors reference ``core/hadamard.py``: ``fwht`` (:23-48), ``inverse_fwht``
(:51-53), ``generate_rht_signs`` (:56-67), ``randomized_hadamard`` (:70-90),
``inverse_randomized_hadamard`` (:93-100) and ``RHTRotation`` (:119-162).
The transforms run in one HIP kernel (``ftq_rht``); device tensors only.
Results are float32 for every input dtype, as in the reference's unfused
path (the sign vector is float32, so torch promotes).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import _lib, _ops


def _validate_power_of_two(d: int, name: str = "d") -> None:
    if d < 1 or (d & (d - 1)) != 0:
        raise ValueError(f"{name} must be a power of 2, got {d}")


def generate_rht_signs(d: int, seed: int = 0, device: torch.device | str = "cpu") -> torch.Tensor:
    """Deterministic +-1 float32 sign vector from the torch CPU generator.

    Same generator call as the reference (core/hadamard.py:56-67), so the
    signs for a given (d, seed) are the reference's.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    signs = torch.randint(0, 2, (d,), generator=gen, dtype=torch.float32, device="cpu") * 2 - 1
    return signs.to(device)


_ONES: dict = {}


def _ones(d: int, device: torch.device) -> torch.Tensor:
    key = (d, str(device))
    t = _ONES.get(key)
    if t is None:
        t = torch.ones(d, dtype=torch.float32, device=device)
        _ONES[key] = t
    return t


def rht_apply(x: torch.Tensor, signs: torch.Tensor, inverse: bool,
              out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """The RHT of the rows of ``x`` (last dim = d) through ``torch.ops.fused_tq.rht``
    (the ``ftq_rht`` kernel)."""
    d = x.shape[-1]
    _validate_power_of_two(d)
    dev = _lib.require_device(x, signs)
    if signs.dtype != torch.float32 or signs.numel() != d:
        raise ValueError("signs must be a float32 vector of length d")
    del dev
    xf = x.contiguous()
    if xf.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        xf = xf.float()
    _lib.dtype_code(out_dtype)
    if not 8 <= d <= 4096:
        raise ValueError(f"head_dim must be a power of two in [8, 4096] for the gfx950 kernels, got {d}")
    return _ops.ops().rht(xf, signs.contiguous(), bool(inverse), out_dtype)


def fwht(x: torch.Tensor) -> torch.Tensor:
    """Orthonormal Fast Walsh-Hadamard Transform of the last dim (float32 out)."""
    _validate_power_of_two(x.shape[-1])
    return rht_apply(x, _ones(x.shape[-1], x.device), inverse=False)


def inverse_fwht(x: torch.Tensor) -> torch.Tensor:
    return fwht(x)


def randomized_hadamard(x: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """y = fwht(x * signs)."""
    return rht_apply(x, signs, inverse=False)


def inverse_randomized_hadamard(y: torch.Tensor, signs: torch.Tensor) -> torch.Tensor:
    """x = fwht(y) * signs."""
    return rht_apply(y, signs, inverse=True)


class RHTRotation(nn.Module):
    """Randomized Hadamard rotation with a persistent sign vector (reference :119-162)."""

    def __init__(self, dim: int, seed: int = 0, device: torch.device | str = "cpu"):
        super().__init__()
        _validate_power_of_two(dim)
        self.dim = dim
        self.register_buffer("signs", generate_rht_signs(dim, seed=seed, device=device))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return randomized_hadamard(x, self.signs)

    def inverse(self, y: torch.Tensor) -> torch.Tensor:
        return inverse_randomized_hadamard(y, self.signs)

    def extra_repr(self) -> str:
        return f"dim={self.dim}, backend=HIP gfx950, storage={self.dim} signs ({self.dim * 4} bytes)"
