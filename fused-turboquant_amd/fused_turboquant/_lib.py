"""Loader for ``libfused_tq.so``: the gfx950 HIP kernels behind the C ABI in
``include/fused_tq.h``.

The library is built in-tree by ``fused-turboquant_amd/build_lib.sh``.  There
is no fallback: if the library or a ROCm device is missing, every hot-path
call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libfused_tq.so")

F32, F16, BF16 = 0, 1, 2
_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_lock = threading.Lock()
_lib = None

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64

# name -> argtypes (all return int status)
SIGNATURES = {
    "ftq_encode": [_vp, _i32, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _vp],
    "ftq_encode_cb": [_vp, _i32, _i64, _i32, _vp, _vp, _i32, _i32, _vp, _vp, _vp],
    "ftq_encode_kv": [_vp, _vp, _i32, _i64, _i32, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp],
    "ftq_codebook_class": [_vp, _i32],
    "ftq_decode": [_vp, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _i32, _vp],
    "ftq_rht": [_vp, _i32, _i64, _i32, _vp, _i32, _vp, _i32, _vp],
}


class FusedTQError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load the HIP library once; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise FusedTQError(
                    f"{LIB_PATH} is missing: build it with fused-turboquant_amd/build_lib.sh "
                    "(or __graft_entry__.build())")
            L = ctypes.CDLL(LIB_PATH)
            L.ftq_last_error.restype = ctypes.c_char_p
            L.ftq_version.restype = ctypes.c_int
            for name, argt in SIGNATURES.items():
                fn = getattr(L, name, None)
                if fn is None:
                    continue
                if argt is not None:
                    fn.argtypes = argt
                    fn.restype = ctypes.c_int
            _lib = L
    return _lib


def check(rc: int) -> None:
    if rc == 0:
        return
    msg = lib().ftq_last_error().decode(errors="replace")
    if rc == -1:
        raise ValueError(msg)
    raise FusedTQError(msg)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; there is no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise FusedTQError(
                "fused_turboquant runs on ROCm devices only (gfx950 HIP kernels); "
                f"got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
