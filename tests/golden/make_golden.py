"""Write the golden fixtures the CPU oracle and the HIP path are checked against.

Run once, in the build container only (the reference tree is not present on the
GPU box):

    python tests/golden/make_golden.py /root/reference/src

It imports the reference's own CPU code (``fused_turboquant.core``) and records
its outputs as data:

* ``codebooks.npz``  -- ``compute_lloyd_max_codebook(d, bits)`` boundaries and
  levels (float64) for d in {64, 128, 256} and bits in {1, 2, 3, 4}
  (reference ``core/lloyd_max.py:24-88``).
* ``signs.npz``      -- ``generate_rht_signs(d, seed)`` for seeds 0, 1, 42
  (reference ``core/hadamard.py:56-67``).
* ``encode.npz``     -- ``TurboQuantMSE(d, bits, seed=42)._encode_unfused`` and
  ``_decode_unfused`` on seeded bf16 inputs (reference
  ``core/quantizer.py:137-160``, ``:191-205``): packed codes, fp16 norms and
  the decoded float32 vectors, plus the pre-quantisation normalised
  coordinates so tie cases can be identified.
* ``fwht.npz``       -- ``fwht`` of a few seeded float32 inputs
  (reference ``core/hadamard.py:23-48``).
* ``rotations.npz``  -- the (D, D) matrices M (``x @ M``) the vLLM rotation
  strategies build: ``planar`` (``vllm_plugin/rotation/planar.py:32-64``),
  ``rotor`` (``rotation/rotor.py:60-166``), ``iso_fast`` and ``iso_full``
  (``rotation/iso.py:65-158``), for D in {64, 128, 256} (rotor also 129 and
  130, the tail cases D mod 3 = 0 and 1), and each strategy's ``[B, D]``
  block coefficients (``rotation/matrix.py:104-124``).

``python tests/golden/make_golden.py [ref_src] rotations`` writes only
``rotations.npz``.

The fixture files are inputs and expected outputs only.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

OUT = os.path.dirname(os.path.abspath(__file__))


def main(ref_src: str) -> None:
    sys.path.insert(0, ref_src)
    from fused_turboquant.core.hadamard import fwht, generate_rht_signs
    from fused_turboquant.core.lloyd_max import compute_lloyd_max_codebook
    from fused_turboquant.core.quantizer import TurboQuantMSE

    dims = (64, 128, 256)
    cb = {}
    for d in dims:
        for bits in (1, 2, 3, 4):
            b, l = compute_lloyd_max_codebook(d, bits)
            cb[f"b_{d}_{bits}"] = np.asarray(b, dtype=np.float64)
            cb[f"l_{d}_{bits}"] = np.asarray(l, dtype=np.float64)
    np.savez_compressed(os.path.join(OUT, "codebooks.npz"), **cb)

    sg = {}
    for d in dims:
        for seed in (0, 1, 42):
            sg[f"s_{d}_{seed}"] = generate_rht_signs(d, seed).numpy().astype(np.float32)
    np.savez_compressed(os.path.join(OUT, "signs.npz"), **sg)

    fw = {}
    g = torch.Generator().manual_seed(7)
    for d in (2, 8, 64, 128, 256):
        x = torch.randn(4, d, generator=g, dtype=torch.float32)
        fw[f"x_{d}"] = x.numpy()
        fw[f"y_{d}"] = fwht(x).numpy()
    np.savez_compressed(os.path.join(OUT, "fwht.npz"), **fw)

    enc = {}
    nvec = 48
    for d in dims:
        for bits in (2, 3, 4):
            g = torch.Generator().manual_seed(1000 + 10 * d + bits)
            scales = torch.exp(0.5 * torch.randn(d, generator=g))
            x = (torch.randn(nvec, d, generator=g) * scales).to(torch.bfloat16)
            # a zero vector and a constant vector exercise the +1e-8 guard and ties
            x[0] = 0
            x[1] = 1
            tq = TurboQuantMSE(d, bits=bits, seed=42)
            ct = tq._encode_unfused(x)
            dec = tq._decode_unfused(ct)
            xr = tq.rotation(x.float())
            nrm = torch.norm(xr, dim=-1, keepdim=True)
            u = xr / (nrm + 1e-8)
            key = f"{d}_{bits}"
            enc[f"x_{key}"] = x.view(torch.int16).numpy().view(np.uint16)
            enc[f"packed_{key}"] = ct.indices.numpy()
            enc[f"norms_{key}"] = ct.norms.view(torch.int16).numpy().view(np.uint16)
            enc[f"dec_{key}"] = dec.numpy()
            enc[f"u_{key}"] = u.numpy()
    # config-1 style input: N(0,1) with 4 outlier channels x10, 4-bit, seed 0
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 128, generator=g)
    x[:, [3, 37, 70, 111]] *= 10
    x = x.to(torch.bfloat16)
    tq = TurboQuantMSE(128, bits=4, seed=0)
    ct = tq._encode_unfused(x)
    enc["x_cfg1"] = x.view(torch.int16).numpy().view(np.uint16)
    enc["packed_cfg1"] = ct.indices.numpy()
    enc["norms_cfg1"] = ct.norms.view(torch.int16).numpy().view(np.uint16)
    enc["dec_cfg1"] = tq._decode_unfused(ct).numpy()
    np.savez_compressed(os.path.join(OUT, "encode.npz"), **enc)
    print("wrote fixtures to", OUT)


def rotations(ref_src: str) -> None:
    """Record the reference's seeded rotation matrices (pure torch on the CPU;
    the strategies' modules import no vLLM)."""
    sys.path.insert(0, ref_src)
    from fused_turboquant.vllm_plugin.rotation import get_rotation

    rot = {}
    for kind, dims in (("planar", (64, 128, 256)), ("rotor", (64, 128, 129, 130, 256)),
                       ("iso_fast", (64, 128, 256)), ("iso_full", (64, 128, 256))):
        strat = get_rotation(kind)
        for d in dims:
            m = strat.build_matrix(d, "cpu").to(torch.float32)
            rot[f"{kind}_{d}"] = m.numpy()
            rot[f"{kind}_{d}_coeffs"] = strat.compute_coeffs(m, strat.block_size).numpy()
    np.savez_compressed(os.path.join(OUT, "rotations.npz"), **rot)
    print("wrote rotations.npz to", OUT)


if __name__ == "__main__":
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    if len(sys.argv) > 2 and sys.argv[2] == "rotations":
        rotations(src)
    else:
        main(src)
        rotations(src)
