"""fused_turboquant on MI355X: TurboQuant KV-cache compression with gfx950 HIP kernels.

Host-side mirror of the reference package's public API
(reference ``src/fused_turboquant/__init__.py:5-32``) for the RHT hot path.
All compute runs in ``libfused_tq.so``; there is no CPU or Triton path.
"""

__version__ = "0.2.0"

from fused_turboquant.core.hadamard import (  # noqa: E402
    RHTRotation,
    fwht,
    generate_rht_signs,
    inverse_fwht,
    inverse_randomized_hadamard,
    randomized_hadamard,
)
from fused_turboquant.core.lloyd_max import LloydMaxQuantizer, compute_lloyd_max_codebook  # noqa: E402
from fused_turboquant.core.quantizer import CompressedTensor, TurboQuantMSE  # noqa: E402

__all__ = [
    "fwht",
    "inverse_fwht",
    "randomized_hadamard",
    "inverse_randomized_hadamard",
    "generate_rht_signs",
    "RHTRotation",
    "LloydMaxQuantizer",
    "compute_lloyd_max_codebook",
    "TurboQuantMSE",
    "CompressedTensor",
]
