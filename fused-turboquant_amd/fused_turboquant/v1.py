"""vLLM v1 ``TURBOQUANT`` slot-format KV cache on gfx950: fused store and
split-K decode attention over the packed slots.

The cache is vLLM's ``uint8[num_blocks, block_size, num_kv_heads, slot]``
(reference ``vllm_plugin/v1_backend.py:171-220``); one slot holds, per
(token, kv head),
``[K codes d*kb/8][K norm f16][V codes d*vb/8][V scale f16][V min f16][pad]``
(``vllm_plugin/triton_inkernel_store.py:38-330``,
``boundary_tq_config.py:66-81``).

* ``v1_store`` replaces the rotation strategy's in-kernel store for
  ``kind=rht`` (``rotation/hadamard.py:43-58`` -> ``_launch_rht``,
  ``triton_inkernel_store.py:554-616``) plus the V pre-rotation of
  ``_launch_store`` (``v1_backend.py:712-749``).
* ``v1_decode_attention`` replaces ``_decode_attention_offset_only``
  (``v1_backend.py:975-1093``): query rotation, ``_tq_decode_stage1_offset``
  (``triton_decode_offset.py:42-442``), the stage-2 LSE merge, the V
  un-rotation and the output cast.
* ``TurboQuantV1Layer`` holds what ``MatrixRotationStrategy.setup_layer``
  keeps per layer (``rotation/matrix.py:34-42``): sorted centroids and their
  midpoints.

The centroid table of vLLM's ``get_centroids(d, bits)``
(``v1_backend.py:624-629``) is not available here; the default is this
library's Lloyd-Max levels for (d, bits) (reference ``core/lloyd_max.py``).
Any sorted float32 table of 2^bits entries may be passed instead.
"""
from __future__ import annotations

import math

import torch

from . import _lib, _ops
from .core.lloyd_max import compute_lloyd_max_codebook

_SIG = {
    "ftq_v1_store": ["vp", "vp", "i32", "i64", "i32", "i32", "vp", "i32", "i32", "i32", "vp", "vp",
                     "i64", "i32", "i64", "i64", "i64", "vp"],
    "ftq_v1_decode_attention": ["vp", "i32", "vp", "i64", "i32", "i64", "i64", "i64", "vp", "i32",
                                "vp", "vp", "i32", "i32", "i32", "i32", "vp", "i32", "i32", "f32",
                                "i32", "i32", "vp", "i64", "vp", "i32", "vp"],
    "ftq_v1_decode_attention_lse": ["vp", "i32", "vp", "i64", "i32", "i64", "i64", "i64", "vp", "i32",
                                    "vp", "vp", "i32", "i32", "i32", "i32", "vp", "i32", "i32", "f32",
                                    "i32", "i32", "vp", "i64", "vp", "i32", "vp", "vp"],
    "ftq_v1_store_rot": ["vp", "vp", "i32", "i64", "i32", "i32", "vp", "i32", "i32", "i32", "vp", "vp",
                         "i64", "i32", "i64", "i64", "i64", "vp", "vp"],
    "ftq_v1_store_blockdiag": ["vp", "vp", "i32", "i64", "i32", "i32", "vp", "i32", "i32", "i32", "vp", "vp",
                               "i64", "i32", "i64", "i64", "i64", "vp", "i32", "vp"],
    "ftq_v1_decode_attention_rot": ["vp", "i32", "vp", "i64", "i32", "i64", "i64", "i64", "vp", "i32",
                                    "vp", "vp", "i32", "i32", "i32", "i32", "vp", "i32", "i32", "f32",
                                    "i32", "i32", "vp", "i64", "vp", "i32", "vp", "vp", "vp"],
}


def _bind():
    import ctypes
    L = _lib.lib()
    if getattr(L, "_v1_bound", False):
        return L
    m = {"vp": ctypes.c_void_p, "i32": ctypes.c_int, "i64": ctypes.c_int64, "f32": ctypes.c_float}
    for name, sig in _SIG.items():
        fn = getattr(L, name)
        fn.argtypes = [m[t] for t in sig]
        fn.restype = ctypes.c_int
    L.ftq_v1_slot_bytes.restype = ctypes.c_int64
    L.ftq_v1_slot_bytes.argtypes = [ctypes.c_int] * 3
    L.ftq_v1_workspace_bytes.restype = ctypes.c_int64
    L.ftq_v1_workspace_bytes.argtypes = [ctypes.c_int] * 4
    L.ftq_v1_default_splits.restype = ctypes.c_int
    L.ftq_v1_default_splits.argtypes = [ctypes.c_int] * 3
    L.ftq_v1_choose_splits.restype = ctypes.c_int
    L.ftq_v1_choose_splits.argtypes = [ctypes.c_int] * 8
    L._v1_bound = True
    return L


def _check_bits(head_dim: int, key_bits: int, value_bits: int, key_fp8: bool = False) -> None:
    """Widths with a store and a decode: K and V both in 1..4 (the
    ``turboquant_k{K}v{V}_nc`` presets and aliases, reference
    ``vllm_plugin/plugin.py:322``), or both 8 -- 8-bit Lloyd-Max keys, or fp8
    keys (``key_fp8``), with 8-bit uniform values (the 8-bit / fp8 boundary
    layers, ``boundary_tq_config.py``)."""
    if head_dim not in (64, 128, 256):
        raise ValueError(f"head_dim must be 64, 128 or 256, got {head_dim}")
    if key_fp8 or key_bits == 8 or value_bits == 8:
        if key_bits != 8 or value_bits != 8:
            raise ValueError("8-bit (and fp8) keys pair with 8-bit values: key_bits = value_bits = 8")
    elif not (1 <= key_bits <= 4) or not (1 <= value_bits <= 4):
        raise ValueError("key_bits and value_bits must be in 1..4 (or both 8)")


def slot_bytes(head_dim: int, key_bits: int, value_bits: int, key_fp8: bool = False) -> int:
    """Bytes of a slot that hold data: key_packed_size + value bytes + 4
    (reference ``boundary_tq_config.py:66-81``); fp8 keys take head_dim bytes
    and no norm."""
    _check_bits(head_dim, key_bits, value_bits, key_fp8)
    kps = head_dim if key_fp8 else head_dim * key_bits // 8 + 2
    return kps + head_dim * value_bits // 8 + 4


def host_preset_bits(key_bits: int, value_bits: int) -> tuple:
    """(K, V) bits of the smallest stock preset whose slot fits a per-K/V bit
    override (reference ``vllm_plugin/plugin.py:390-402``)."""
    if key_bits <= 3 and value_bits <= 3:
        return 3, 3
    if key_bits <= 3 and value_bits <= 4:
        return 3, 4
    return 4, 4


def slot_size(head_dim: int, key_bits: int, value_bits: int, boundary_protect: bool = False) -> int:
    """Last-dim size of the cache: the host preset's slot bytes rounded up to a
    power of two, at least 2*head_dim bf16 elements worth when boundary
    protection shares the allocation (reference ``v1_backend.py:171-209``)."""
    hk, hv = host_preset_bits(key_bits, value_bits)
    raw = slot_bytes(head_dim, hk, hv)
    if boundary_protect:
        raw = max(raw, 2 * head_dim)
    return 1 << (raw - 1).bit_length()


def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int, head_size: int,
                       key_bits: int = 4, value_bits: int = 4) -> tuple:
    """(num_blocks, block_size, num_kv_heads, slot) (reference ``v1_backend.py:211-220``)."""
    return (num_blocks, block_size, num_kv_heads, slot_size(head_size, key_bits, value_bits))


def default_centroids(head_dim: int, bits: int, device=None) -> torch.Tensor:
    """Sorted float32 Lloyd-Max levels for the coordinate distribution at head_dim."""
    _, levels = compute_lloyd_max_codebook(head_dim, bits)
    c = torch.as_tensor(levels, dtype=torch.float32)
    return torch.sort(c).values.to(device) if device is not None else torch.sort(c).values


def midpoints_of(centroids: torch.Tensor) -> torch.Tensor:
    """(c[i] + c[i+1]) / 2 of the sorted table (reference ``rotation/matrix.py:38-41``)."""
    c = torch.sort(centroids.to(torch.float32)).values
    return (c[:-1] + c[1:]) / 2


def _strides(kv_cache: torch.Tensor):
    if kv_cache.dtype != torch.uint8 or kv_cache.dim() != 4:
        raise ValueError("kv_cache must be uint8 [num_blocks, block_size, num_kv_heads, slot]")
    if kv_cache.stride(3) != 1:
        raise ValueError("kv_cache slot bytes must be contiguous")
    return kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2)


# bits of the C ABI's v_rotate / v_flags word (FTQ_V1_* in fused_tq.h)
VROT, VLLOYD, KFP8, FP32 = 1, 2, 4, 8


def _v_flags(v_rotate: bool, v_lloyd_max: bool, key_fp8: bool = False, fp32: bool = False) -> int:
    return ((VROT if (v_rotate or v_lloyd_max) else 0) | (VLLOYD if v_lloyd_max else 0)
            | (KFP8 if key_fp8 else 0) | (FP32 if fp32 else 0))


_OPERANDS = ("f16", "fp32")


def planar_rotation(head_dim: int, seed: int = 42, device="cpu") -> torch.Tensor:
    """Rotation matrix M (x M, float32 [d, d]) of the planar strategy
    (reference ``vllm_plugin/rotation/planar.py:32-67``,
    ``core/planar.py:48-68``): pair p of coordinates (2p, 2p + 1) is turned by
    an angle theta_p = 2 pi U[0, 1) from a CPU ``torch.Generator`` seeded
    ``seed``; block p of M is [[cos, sin], [-sin, cos]], so
    x M = [cos x0 - sin x1, sin x0 + cos x1] per pair."""
    if head_dim % 2:
        raise ValueError("planar rotation needs an even head_dim")
    n = head_dim // 2
    gen = torch.Generator(device="cpu").manual_seed(seed)
    theta = torch.rand(n, generator=gen, device="cpu") * (2.0 * math.pi)
    c, sn = theta.cos().to(torch.float32), theta.sin().to(torch.float32)
    m = torch.zeros(head_dim, head_dim, dtype=torch.float32)
    i = torch.arange(n)
    m[2 * i, 2 * i] = c
    m[2 * i, 2 * i + 1] = sn
    m[2 * i + 1, 2 * i] = -sn
    m[2 * i + 1, 2 * i + 1] = c
    return m.to(device)


def rotor_rotation(head_dim: int, seed: int = 42, device="cpu") -> torch.Tensor:
    """Rotation matrix M (x M, float32 [d, d]) of the rotor strategy (reference
    ``vllm_plugin/rotation/rotor.py:60-166``): coordinates in groups of 3, each
    turned by the 3x3 matrix of a Cl(3,0) rotor (s, p12, p13, p23) =
    (cos(a/2), sin(a/2) b) with b a unit vector from ``randn`` and a = 2 pi
    U[0, 1), both drawn for ceil(d/3) groups from a CPU generator seeded
    ``seed``; d mod 3 = 2 trailing coordinates take a Givens turn by a third
    draw, 1 is left alone.  Blocks are built in column form and M is their
    transpose."""
    D = head_dim
    n, r = D // 3, D % 3
    npad = (D + 2) // 3
    gen = torch.Generator(device="cpu").manual_seed(seed)
    m = torch.zeros(D, D, dtype=torch.float32)
    if n > 0:
        b = torch.randn(npad, 3, generator=gen, dtype=torch.float32)[:n]
        b = b / b.norm(dim=-1, keepdim=True).clamp(min=1e-8)
        a = (torch.rand(npad, generator=gen, dtype=torch.float32) * (2.0 * math.pi))[:n]
        h = a / 2
        sc = torch.cos(h)
        sh = torch.sin(h)
        p12, p13, p23 = sh * b[:, 0], sh * b[:, 1], sh * b[:, 2]
        s2, q12, q13, q23 = sc * sc, p12 * p12, p13 * p13, p23 * p23
        rows = [
            [s2 - q12 - q13 + q23, 2 * sc * p12 - 2 * p13 * p23, 2 * sc * p13 + 2 * p12 * p23],
            [-2 * sc * p12 - 2 * p13 * p23, s2 - q12 + q13 - q23, 2 * sc * p23 - 2 * p12 * p13],
            [-2 * sc * p13 + 2 * p12 * p23, -2 * sc * p23 - 2 * p12 * p13, s2 + q12 - q13 - q23],
        ]
        for i in range(3):
            for j in range(3):
                m[3 * torch.arange(n) + i, 3 * torch.arange(n) + j] = rows[i][j]
    t = 3 * n
    if r == 1:
        m[t, t] = 1.0
    elif r == 2:
        th = torch.rand(1, generator=gen, dtype=torch.float32).item() * (2.0 * math.pi)
        c, sn = math.cos(th), math.sin(th)
        m[t, t], m[t, t + 1], m[t + 1, t], m[t + 1, t + 1] = c, -sn, sn, c
    return m.T.contiguous().to(device)


def _unit_quaternions(n: int, seed: int) -> torch.Tensor:
    """n unit quaternions (w, x, y, z): ``randn(n, 4)`` from a CPU generator
    seeded ``seed``, each divided by max(norm, 1e-8)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(n, 4, generator=gen, dtype=torch.float32)
    return q / q.norm(dim=-1, keepdim=True).clamp(min=1e-8)


def _quat_mat(q: torch.Tensor, right: bool) -> torch.Tensor:
    """[n, 4, 4] column-form matrices of v -> q v (right=False) or v -> v q
    (right=True) under the Hamilton product, components (w, x, y, z)."""
    w, x, y, z = q.unbind(-1)
    if right:
        rows = ((w, -x, -y, -z), (x, w, z, -y), (y, -z, w, x), (z, y, -x, w))
    else:
        rows = ((w, -x, -y, -z), (x, w, -z, y), (y, z, w, -x), (z, -y, x, w))
    return torch.stack([torch.stack(r, dim=-1) for r in rows], dim=-2)


def iso_rotation(head_dim: int, full: bool = False, seed: int = 42, device="cpu") -> torch.Tensor:
    """Rotation matrix M (x M, float32 [d, d]) of the IsoQuant strategies
    (reference ``vllm_plugin/rotation/iso.py:65-158``): coordinates in groups
    of 4, each group a quaternion v turned to q_L v (``iso_fast``) or
    q_L v conj(q_R) (``iso_full``), q_L drawn with ``seed`` and q_R with
    ``seed + 10000``; d is padded to a multiple of 4 and M cropped back.
    Blocks are built in column form and M is their transpose."""
    D = head_dim
    dp = (D + 3) // 4 * 4
    n = dp // 4
    blk = _quat_mat(_unit_quaternions(n, seed), right=False)
    if full:
        qr = _unit_quaternions(n, seed + 10000) * torch.tensor([1.0, -1.0, -1.0, -1.0])
        r = _quat_mat(qr, right=True)
        # the 4x4 block product L R, summed k = 0..3 in order in fp32 (no fused
        # multiply-add), so the result does not depend on the host's BLAS
        acc = blk[:, :, 0, None] * r[:, None, 0, :]
        for k in range(1, 4):
            acc = acc + blk[:, :, k, None] * r[:, None, k, :]
        blk = acc
    m = torch.zeros(dp, dp, dtype=torch.float32)
    g = torch.arange(n)
    for i in range(4):
        for j in range(4):
            m[4 * g + i, 4 * g + j] = blk[:, i, j]
    return m.T[:D, :D].contiguous().to(device)


# block size of each block-diagonal strategy (reference rotation/*.py block_size)
BLOCK_SIZES = {"planar": 2, "rotor": 3, "iso_fast": 4, "iso_full": 4}


def rotation_matrix(kind: str, head_dim: int, device="cpu") -> torch.Tensor:
    """M of a registered matrix strategy (``TURBOQUANT_KIND``) at head_dim."""
    if kind == "planar":
        return planar_rotation(head_dim, device=device)
    if kind == "rotor":
        return rotor_rotation(head_dim, device=device)
    if kind in ("iso_fast", "iso_full"):
        return iso_rotation(head_dim, full=(kind == "iso_full"), device=device)
    raise ValueError(f"no rotation matrix for kind {kind!r}")


def block_coeffs(m: torch.Tensor, block: int) -> torch.Tensor:
    """[B, D] coefficients of a block-diagonal M with B x B blocks:
    coeffs[k][d] = M[(d // B) B + k][d], 0 where that row is past D, so
    (x M)[d] = sum_k x[(d // B) B + k] coeffs[k][d] (reference
    ``rotation/matrix.py:104-124``)."""
    D = m.shape[-1]
    d = torch.arange(D, device=m.device)
    src = (d // block * block)[None, :] + torch.arange(block, device=m.device)[:, None]
    ok = src < D
    c = m[torch.where(ok, src, torch.zeros_like(src)), d[None, :].expand(block, D)]
    return (c * ok.to(m.dtype)).contiguous()


def _rotation_arg(rotation: torch.Tensor, d: int, dev) -> torch.Tensor:
    if rotation.shape != (d, d):
        raise ValueError("rotation must be a [head_dim, head_dim] matrix")
    return rotation.to(device=dev, dtype=torch.float32).contiguous()


def v1_store(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
             slot_mapping: torch.Tensor, midpoints: torch.Tensor, key_bits: int,
             value_bits: int, v_rotate: bool = False, v_lloyd_max: bool = False,
             rotation: torch.Tensor | None = None, coeffs: torch.Tensor | None = None,
             key_fp8: bool = False) -> None:
    """Quantise ``key``/``value`` [n, Hkv, d] into their slots (``slot_mapping`` [n]
    int64; negative entries are skipped).  ``key_fp8`` (key_bits = value_bits
    = 8): K stored as fp8 e4m3fn, no norm, ``midpoints`` unused (reference
    ``triton_inkernel_store.py:59-83``).  ``v_lloyd_max`` (implies
    ``v_rotate``): 4-bit V takes Lloyd-Max codes against the K midpoints and its
    norm in the scale field (reference ``triton_inkernel_store.py:159-200``);
    other V widths keep the uniform codes.  ``coeffs`` ([B, d] float32, B in
    2/3/4): a block-diagonal rotation given by its block coefficients
    (``block_coeffs``), O(B d) per vector (reference ``_fused_store_block_diag``,
    ``triton_inkernel_store.py:649-860``); ``rotation``: any d x d matrix, O(d^2)."""
    n, hkv, d = key.shape
    _check_bits(d, key_bits, value_bits, key_fp8)
    if value.shape != key.shape:
        raise ValueError("key and value shapes differ")
    nb, bs, hk2, slot = kv_cache.shape
    if hk2 != hkv:
        raise ValueError("kv_cache num_kv_heads does not match key")
    if slot < slot_bytes(d, key_bits, value_bits, key_fp8):
        raise ValueError("kv_cache slot is smaller than the slot bytes for these bits")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != n:
        raise ValueError("slot_mapping must be int64 with one entry per token")
    if midpoints is None or key_fp8:
        midpoints = torch.zeros(1, dtype=torch.float32, device=key.device)
    elif midpoints.numel() != (1 << key_bits) - 1:
        raise ValueError("midpoints must have 2^key_bits - 1 entries")
    dev = _lib.require_device(key, value, kv_cache, slot_mapping, midpoints)
    k = key.contiguous()
    if k.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        k = k.float()
    v = value.to(k.dtype).contiguous()
    _strides(kv_cache)
    mids = midpoints.to(torch.float32).contiguous()
    cf = rot = None
    if coeffs is not None:  # block-diagonal strategy: planar (B=2), rotor (3), iso (4)
        if coeffs.dim() != 2 or coeffs.shape[1] != d or coeffs.shape[0] not in (2, 3, 4):
            raise ValueError("coeffs must be [B, head_dim] with B in 2, 3, 4")
        cf = coeffs.to(device=dev, dtype=torch.float32).contiguous()
    elif rotation is not None:  # any d x d matrix: x M in the kernel
        rot = _rotation_arg(rotation, d, dev)
    _ops.ops().v1_store(k, v, kv_cache, slot_mapping.contiguous(), mids, key_bits, value_bits,
                        _v_flags(v_rotate, v_lloyd_max, key_fp8), rot, cf)


def default_splits(batch: int, num_kv_heads: int, max_seq_len: int, num_q_heads: int | None = None,
                   head_dim: int | None = None, key_bits: int | None = None, value_bits: int | None = None,
                   v_flags: int = 0) -> int:
    """Split-K factor of the decode.  With the head geometry and widths
    (``num_q_heads``, ``head_dim``, ``key_bits``, ``value_bits``, and the
    ``v_flags`` bits of the call) it is sized to the kernel that runs: for the
    matrix-core kernels the most splits whose workgroups the GPU holds at once
    (``ftq_v1_choose_splits``); without them, ``ftq_v1_default_splits``."""
    if None not in (num_q_heads, head_dim, key_bits, value_bits):
        return int(_bind().ftq_v1_choose_splits(batch, num_q_heads, num_kv_heads, head_dim, key_bits,
                                                value_bits, v_flags, max_seq_len))
    return int(_bind().ftq_v1_default_splits(batch, num_kv_heads, max_seq_len))


def workspace_bytes(batch: int, num_q_heads: int, head_dim: int, num_splits: int) -> int:
    return int(_bind().ftq_v1_workspace_bytes(batch, num_q_heads, head_dim, num_splits))


def v1_decode_attention(query: torch.Tensor, kv_cache: torch.Tensor, block_table: torch.Tensor,
                        seq_lens: torch.Tensor, centroids: torch.Tensor, key_bits: int,
                        value_bits: int, scale: float | None = None, v_rotate: bool = False,
                        v_lloyd_max: bool = False,
                        kv_start: torch.Tensor | None = None, num_splits: int | None = None,
                        max_seq_len: int | None = None, out: torch.Tensor | None = None,
                        workspace: torch.Tensor | None = None, lse: torch.Tensor | None = None,
                        rotation: torch.Tensor | None = None, sorted_centroids: bool = False,
                        key_fp8: bool = False, operands: str = "f16") -> torch.Tensor:
    """query [B, Hq, d] -> [B, Hq, d] (query dtype unless ``out`` is given).

    Attends positions [kv_start[b], seq_lens[b]) of block-table row b
    (``kv_start`` None = 0, reference ``triton_decode_offset.py:95-106``).
    ``num_splits`` defaults to a value that fills the GPU (pass ``max_seq_len``
    to size it without reading ``block_table``'s width); ``workspace`` (uint8,
    >= ``workspace_bytes``) may be preallocated for graph capture.  ``lse``
    (float32 [B, Hq]) receives each row's natural-log log-sum-exp of the
    scaled scores (-inf for a row with no positions).  ``sorted_centroids``:
    the table is already sorted (skips the sort, e.g. for graph capture).
    ``key_fp8``: the keys are fp8 e4m3fn (``centroids`` unused).
    ``operands``: ``"f16"`` (default) runs head_dim 128 with 2-4 bit codes on
    the matrix-core kernels (f16 operands, fp32 accumulation); ``"fp32"``
    keeps every product in fp32 on the VALU, the reference's arithmetic.
    Head dims 64 and 256, 1- and 8-bit codes and fp8 keys always take the
    fp32 kernel.
    """
    B, hq, d = query.shape
    _check_bits(d, key_bits, value_bits, key_fp8)
    if operands not in _OPERANDS:
        raise ValueError(f"operands must be one of {_OPERANDS}, got {operands!r}")
    nb, bs, hkv, slot = kv_cache.shape
    if slot < slot_bytes(d, key_bits, value_bits, key_fp8):
        raise ValueError("kv_cache slot is smaller than the slot bytes for these bits")
    if block_table.dtype != torch.int32 or seq_lens.dtype != torch.int32:
        raise ValueError("block_table and seq_lens must be int32")
    if block_table.dim() != 2 or block_table.shape[0] != B or seq_lens.numel() != B:
        raise ValueError("block_table must be [B, max_blocks] and seq_lens [B]")
    if kv_start is not None and (kv_start.dtype != torch.int32 or kv_start.numel() != B):
        raise ValueError("kv_start must be int32 [B]")
    if centroids is None or key_fp8:
        centroids = torch.zeros(1, dtype=torch.float32, device=query.device)
        sorted_centroids = True
    elif centroids.numel() != (1 << key_bits):
        raise ValueError("centroids must have 2^key_bits entries")
    if lse is not None and (lse.dtype != torch.float32 or lse.numel() != B * hq or not lse.is_contiguous()):
        raise ValueError("lse must be a contiguous float32 tensor of B * num_q_heads entries")
    tensors = [query, kv_cache, block_table, seq_lens, centroids] + ([kv_start] if kv_start is not None else [])
    tensors += [lse] if lse is not None else []
    dev = _lib.require_device(*tensors)
    q = query.contiguous()
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        q = q.float()
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    flags = _v_flags(v_rotate, v_lloyd_max, key_fp8, operands == "fp32")
    if num_splits is None:
        msl = max_seq_len if max_seq_len is not None else block_table.shape[1] * bs
        num_splits = default_splits(B, hkv, msl, hq, d, key_bits, value_bits, flags)
    if out is None:
        out = torch.empty(B, hq, d, dtype=q.dtype, device=dev)
    need = workspace_bytes(B, hq, d, num_splits)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    _strides(kv_cache)
    cent = centroids.to(torch.float32)
    if not sorted_centroids:
        cent = torch.sort(cent).values
    ks = kv_start.contiguous() if kv_start is not None else None
    rot = _rotation_arg(rotation, d, dev) if rotation is not None else None  # q M, and o M^T with v_rotate
    _ops.ops().v1_decode_attention(q, kv_cache, block_table.contiguous(), seq_lens.contiguous(), ks,
                                   cent.contiguous(), key_bits, value_bits, float(scale),
                                   flags, int(num_splits), workspace, out, lse, rot)
    return out


class TurboQuantV1Layer:
    """Per-layer state of the v1 backend for ``kind=rht``: sorted centroids and
    midpoints (reference ``rotation/matrix.py:34-42``), bit widths and the
    V-rotation switch (``TURBOQUANT_V_ROTATE``, ``v1_backend.py:733-740``)."""

    def __init__(self, head_dim: int, key_bits: int, value_bits: int, v_rotate: bool = False,
                 centroids: torch.Tensor | None = None, device="cuda", v_lloyd_max: bool = False,
                 kind: str = "rht", rotation: torch.Tensor | None = None, key_fp8: bool = False,
                 operands: str = "f16"):
        _check_bits(head_dim, key_bits, value_bits, key_fp8)
        if operands not in _OPERANDS:
            raise ValueError(f"operands must be one of {_OPERANDS}, got {operands!r}")
        self.head_dim = head_dim
        self.key_bits = key_bits
        self.value_bits = value_bits
        self.key_fp8 = bool(key_fp8)
        self.operands = operands
        self.v_lloyd_max = bool(v_lloyd_max)
        self.v_rotate = bool(v_rotate) or self.v_lloyd_max
        if self.key_fp8:  # fp8 keys: no codebook (the 8-bit V is uniform)
            self.centroids = torch.zeros(1, dtype=torch.float32, device=device)
            self.midpoints = self.centroids
        else:
            c = centroids if centroids is not None else default_centroids(head_dim, key_bits)
            if c.numel() != (1 << key_bits):
                raise ValueError("centroids must have 2^key_bits entries")
            self.centroids = torch.sort(c.to(torch.float32)).values.to(device)
            self.midpoints = midpoints_of(self.centroids)
        # rotation strategy (TURBOQUANT_KIND): rht = the kernels' own H/sqrt(d);
        # planar = a matrix x M applied in the kernels; a caller's matrix the same
        self.kind = kind
        self.coeffs = None  # [B, d] block coefficients of a block-diagonal strategy (the store's form)
        if rotation is not None:
            self.rotation = rotation.to(device=device, dtype=torch.float32).contiguous()
        elif kind == "rht":
            self.rotation = None
        elif kind in BLOCK_SIZES:
            m = rotation_matrix(kind, head_dim)
            self.rotation = m.to(device)
            self.coeffs = block_coeffs(m, BLOCK_SIZES[kind]).to(device)
        else:
            raise ValueError(f"rotation kind {kind!r}: rht, planar, rotor, iso_fast, iso_full "
                             "or an explicit matrix")

    def kv_cache_shape(self, num_blocks: int, block_size: int, num_kv_heads: int) -> tuple:
        if self.key_bits == 8:  # 8-bit formats live in boundary-layer slots: the raw bytes, rounded up
            raw = slot_bytes(self.head_dim, 8, 8, self.key_fp8)
            return (num_blocks, block_size, num_kv_heads, 1 << (raw - 1).bit_length())
        return get_kv_cache_shape(num_blocks, block_size, num_kv_heads, self.head_dim,
                                  self.key_bits, self.value_bits)

    def store(self, key, value, kv_cache, slot_mapping) -> None:
        v1_store(key, value, kv_cache, slot_mapping, self.midpoints, self.key_bits,
                 self.value_bits, self.v_rotate, self.v_lloyd_max,
                 rotation=self.rotation if self.coeffs is None else None, coeffs=self.coeffs,
                 key_fp8=self.key_fp8)

    def decode(self, query, kv_cache, block_table, seq_lens, **kw) -> torch.Tensor:
        return v1_decode_attention(query, kv_cache, block_table, seq_lens, self.centroids,
                                   self.key_bits, self.value_bits, v_rotate=self.v_rotate,
                                   v_lloyd_max=self.v_lloyd_max, rotation=self.rotation,
                                   sorted_centroids=True, key_fp8=self.key_fp8,
                                   **{"operands": self.operands, **kw})
