"""``torch.ops.fused_tq``: the PyTorch operators over the C ABI.

``libfused_tq_torch.so`` (built next to ``libfused_tq.so`` by
``build_lib.sh``) registers the operator schemas and their ROCm
implementations (``csrc/ftq_torch_ops.cpp``); each checks its tensors and
calls the C entry point on the tensors' current HIP stream.  This module
loads it and registers the shape-only ("fake") implementations that let
``torch.compile`` and other tracers see through the calls without running a
kernel.  The package's functions call these operators; there is no fallback:
a missing library raises.
"""
from __future__ import annotations

import os
import threading

import torch

from . import _lib

OPS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfused_tq_torch.so")

_lock = threading.Lock()
_loaded = False


def _register_fakes() -> None:
    lib = "fused_tq::"

    @torch.library.register_fake(lib + "encode")
    def _encode(x, signs, boundaries, bits, codebook_class):
        d = x.shape[-1]
        return (x.new_empty((*x.shape[:-1], d * bits // 8), dtype=torch.uint8),
                x.new_empty(x.shape[:-1], dtype=torch.float16))

    @torch.library.register_fake(lib + "encode_kv")
    def _encode_kv(k, v, signs, boundaries, bits, codebook_class):
        d = k.shape[-1]
        return (k.new_empty((*k.shape[:-1], d * bits // 8), dtype=torch.uint8),
                k.new_empty(k.shape[:-1], dtype=torch.float16),
                v.new_empty((*v.shape[:-1], d * bits // 8), dtype=torch.uint8),
                v.new_empty(v.shape[:-1], dtype=torch.float16))

    @torch.library.register_fake(lib + "decode")
    def _decode(packed, norms, levels, signs, bits, d, out_dtype):
        return packed.new_empty((*norms.shape, d), dtype=out_dtype)

    @torch.library.register_fake(lib + "rht")
    def _rht(x, signs, inverse, out_dtype):
        return x.new_empty(x.shape, dtype=out_dtype)

    # operators that only write their (a!) arguments
    for name in ("paged_store", "paged_decode_attention", "v1_store", "v1_decode_attention", "raw_store",
                 "raw_decode_attention"):
        torch.library.register_fake(lib + name)(lambda *args, **kwargs: None)


def ops():
    """``torch.ops.fused_tq`` with the operator library loaded (once)."""
    global _loaded
    if not _loaded:
        with _lock:
            if not _loaded:
                if not os.path.exists(OPS_PATH):
                    raise _lib.FusedTQError(
                        f"{OPS_PATH} is missing: build it with fused-turboquant_amd/build_lib.sh "
                        "(or __graft_entry__.build())")
                _lib.lib()  # the C library the operators call into
                torch.ops.load_library(OPS_PATH)
                _register_fakes()
                _loaded = True
    return torch.ops.fused_tq
