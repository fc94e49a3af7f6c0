"""Lloyd-Max codebook for Beta-distributed rotated coordinates.

Host-side setup, computed once per (dim, bits): the grid Lloyd-Max iteration
of reference ``core/lloyd_max.py:24-88`` (float64 numpy), cached as in
``:144-152``.  ``LloydMaxQuantizer`` mirrors ``:91-141``; its
``quantize`` / ``dequantize`` helpers are plain torch ops on whatever device
the tensors live on -- the hot path never calls them (the fused encode and
decode kernels do the bucketize and the level lookup themselves).
"""
from __future__ import annotations

import math
from functools import lru_cache

import numpy as np
import torch


def compute_lloyd_max_codebook(dim: int, bits: int, max_iterations: int = 300,
                               num_grid_points: int = 50000):
    """Returns ``(boundaries[2^bits + 1], levels[2^bits])`` as float64 numpy arrays."""
    num_levels = 1 << bits
    exponent = (dim - 3) / 2.0
    sigma = 1.0 / math.sqrt(dim)
    lo = max(-1.0, -6.0 * sigma)
    hi = min(1.0, 6.0 * sigma)
    grid = np.linspace(lo, hi, num_grid_points)
    weights = np.maximum(1.0 - grid ** 2, 0.0) ** exponent
    weights /= weights.sum()
    boundaries = np.interp(np.linspace(0, 1, num_levels + 1), np.cumsum(weights), grid)
    boundaries[0] = lo
    boundaries[-1] = hi
    levels = np.zeros(num_levels)

    def update_levels() -> None:
        for i in range(num_levels):
            upper_ok = grid <= boundaries[i + 1] if i == num_levels - 1 else grid < boundaries[i + 1]
            mask = (grid >= boundaries[i]) & upper_ok
            w = weights[mask]
            levels[i] = (np.average(grid[mask], weights=w) if w.sum() > 0
                         else (boundaries[i] + boundaries[i + 1]) / 2.0)

    update_levels()
    for _ in range(max_iterations):
        boundaries[1:num_levels] = [(levels[i - 1] + levels[i]) / 2.0 for i in range(1, num_levels)]
        update_levels()
    return boundaries, levels


@lru_cache(maxsize=32)
def _get_cached_codebook(dim: int, bits: int, max_iterations: int = 300,
                         num_grid_points: int = 50000):
    return compute_lloyd_max_codebook(dim, bits, max_iterations, num_grid_points)


CB_ANY, CB_SYMMETRIC = 0, 1  # FTQ_CB_ANY / FTQ_CB_SYMMETRIC of the C ABI


def codebook_class(boundaries, bits: int) -> int:
    """Host-side class of a float32 codebook, as the C ABI's ``ftq_codebook_class``
    computes it: ``CB_SYMMETRIC`` when sorted, ``B[2^bits - j] == -B[j]`` for every
    interior j but the middle one, and ``|B[mid]| < B[mid + 1]``; else ``CB_ANY``.
    The encoder's symmetric kernel searches |t| over the positive thresholds."""
    b = np.asarray(boundaries, dtype=np.float32)
    if b.shape != ((1 << bits) + 1,) or not np.all(b[:-1] <= b[1:]):
        return CB_ANY
    mid = 1 << (bits - 1)
    if not abs(b[mid]) < b[mid + 1]:
        return CB_ANY
    for k in range(1, mid):
        if not b[mid + k] == -b[mid - k]:
            return CB_ANY
    return CB_SYMMETRIC


class LloydMaxQuantizer:
    """Precomputed Lloyd-Max scalar quantizer, shared by all layers/heads/tokens."""

    def __init__(self, dim: int, bits: int = 4, device: torch.device | str = "cpu",
                 max_iterations: int = 300, num_grid_points: int = 50000):
        self.dim = dim
        self.bits = bits
        self.num_levels = 1 << bits
        b, l = _get_cached_codebook(dim, bits, max_iterations, num_grid_points)
        self.boundaries = torch.tensor(b, dtype=torch.float32, device=device)
        self.levels = torch.tensor(l, dtype=torch.float32, device=device)
        self.levels_host = np.asarray(l, dtype=np.float32)  # host copy (kernel set-up decisions)
        self.codebook_class = codebook_class(np.asarray(b, dtype=np.float32), bits)

    def quantize(self, x: torch.Tensor) -> torch.Tensor:
        idx = torch.bucketize(x, self.boundaries) - 1
        return idx.clamp(0, self.num_levels - 1).to(torch.uint8)

    def dequantize(self, indices: torch.Tensor) -> torch.Tensor:
        return self.levels[indices.long()]

    def to(self, device: torch.device | str) -> "LloydMaxQuantizer":
        self.boundaries = self.boundaries.to(device)
        self.levels = self.levels.to(device)
        return self
