"""Shared byte checks of vLLM v1 slot stores against the CPU oracle."""
import numpy as np

from oracle import tq_oracle as O


def check_v_region(got, want, st, ok, blk, off, geo, vrot, dtype, vb, lloyd=False, tag=""):
    """V codes, V scale and V min of every stored (token, kv head) equal the
    oracle's, except in the vectors whose bytes the float32 order of the V
    pre-rotation can change (``O.v1_v_tie_vectors``: the reference rotates V
    by a dense float32 product, v1_backend.py:736-740, whose summation order is
    its GEMM's); the padding after them is byte-exact.  Returns the number of
    (token, head) vectors that differ and the number flagged."""
    kps, raw = geo["kps"], geo["raw"]
    g = got[blk, off, :, kps:raw]
    w = want[blk, off, :, kps:raw]
    diff = np.any(g != w, axis=-1)
    if vrot:
        flagged = O.v1_v_tie_vectors(st["vrot"][ok], dtype, vb, v_lloyd_max=lloyd)
    else:
        flagged = np.zeros(diff.shape, bool)
    bad = diff & ~flagged
    assert not bad.any(), (tag, int(bad.sum()), np.argwhere(bad)[:4])
    assert np.array_equal(got[..., raw:], want[..., raw:]), tag
    if vrot:
        print(f"[{tag}] V rotation ties: {int(diff.sum())} vectors differ, {int(flagged.sum())} flagged "
              f"of {diff.size}")
    return int(diff.sum()), int(flagged.sum())
