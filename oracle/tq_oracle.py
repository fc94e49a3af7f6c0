"""CPU oracle for the fused-turboquant KV-cache hot path (TEST INFRASTRUCTURE).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``fused_turboquant``) never calls into it and has
no CPU fallback.

It restates, in numpy, the reference's unfused PyTorch algorithm:

* ``fwht`` / ``rht`` / ``inverse_rht`` -- reference ``core/hadamard.py:23-48``
  (butterfly order h = 1, 2, 4, ...; pairs ``[a+b, a-b]``; final ``* d**-0.5``
  rounded to float32) and ``:70-100`` (sign flip before / after).
* ``lloyd_max_codebook`` -- reference ``core/lloyd_max.py:24-88`` (grid
  Lloyd-Max on the Beta coordinate density, 300 iterations, float64).
* ``quantize`` -- reference ``core/lloyd_max.py:121-132``
  (``bucketize(right=False) - 1`` clamped to ``[0, 2^b - 1]``).
* ``pack_*`` / ``unpack_*`` -- reference ``core/packing.py:14-128``.
* ``encode`` / ``decode`` -- reference ``core/quantizer.py:137-160`` and
  ``:191-205`` (``TurboQuantMSE._encode_unfused`` / ``_decode_unfused``).
* ``dense_decode_attention`` -- the semantics of library-format decode
  attention, reference ``vllm_plugin/attention_impl.py:431-521`` and
  ``kernels/triton_flash_decode.py:66-221``: softmax(q . K^ * scale) . V^ with
  K^, V^ the decoded cache, computed in float64.
* ``v1_*`` -- the vLLM v1 ``TURBOQUANT`` slot format: store
  ``vllm_plugin/triton_inkernel_store.py:38-440`` and decode stage 1/2
  ``vllm_plugin/triton_decode_offset.py:42-442`` + ``v1_backend.py:975-1093``.

Pinning (each check lives in ``tests/test_oracle.py``):

* fwht: the reference's d=2 known answer, an explicit Sylvester matrix product,
  involution, and the reference's own outputs (``tests/golden/fwht.npz``).
* codebook: the reference's own outputs for d in {64,128,256} x bits in
  {1,2,3,4} (``tests/golden/codebooks.npz``), plus sortedness / symmetry.
* signs: the reference's own outputs (``tests/golden/signs.npz``).
* quantize/pack: brute force over every 3-bit group and random bytes, and the
  reference's codes (``tests/golden/encode.npz``).
* encode/decode: the reference's own codes, fp16 norms and decoded vectors
  (``tests/golden/encode.npz``).
* dense attention: an independent float64 computation in the test of the
  rotated-domain identity <q, RHT^-1 c> = <RHT q, c>, and the reference's
  structure (softmax over masked scores).
* v1 store/decode: parity unpinned against vLLM (vLLM's ``get_centroids`` and
  stage-2 kernel are not in the reference tree); pinned by closed forms (LSE
  merge == single softmax, uniform quantiser error bound, Hadamard matrix).
* raw_* (boundary-layer fp16 slots, ``vllm_plugin/v1_backend.py:1449-1545``,
  ``triton_boundary_attn.py:28-219``): the store is numpy's float16 rounding
  (IEEE round to nearest even, as torch's ``.to(float16)``); the attention is
  float64 softmax attention, checked against an independent dense computation
  over the K/V arrays before they enter the cache.
* v1_hybrid_decode_attention (deferred-prefill decode,
  ``vllm_plugin/v1_backend.py:1095-1277``): one float64 softmax over the union
  of the fp16 prefix (sequence 0) and the dequantised slots in [P, seq_len);
  the reference's two phases and log-sum-exp merge equal it in closed form.
  Checked against a two-phase computation (``v1_decode_attention`` with
  ``kv_start`` plus dense attention over the prefix, merged by their LSEs).
"""
from __future__ import annotations

import math

import numpy as np

# --------------------------------------------------------------------------
# Hadamard transforms  (reference core/hadamard.py:23-100)
# --------------------------------------------------------------------------


def _check_pow2(d: int) -> None:
    if d < 1 or (d & (d - 1)) != 0:
        raise ValueError(f"d must be a power of 2, got {d}")


def fwht_unscaled(x: np.ndarray) -> np.ndarray:
    """Butterflies only, float32, h = 1, 2, 4, ... (reference hadamard.py:37-47)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    _check_pow2(d)
    lead = x.shape[:-1]
    h = 1
    while h < d:
        v = x.reshape(*lead, d // (2 * h), 2, h)
        a = v[..., 0, :]
        b = v[..., 1, :]
        x = np.stack([a + b, a - b], axis=-2).reshape(*lead, d)
        h *= 2
    return x


def fwht_scale(d: int) -> np.float32:
    """``d ** -0.5`` as the float32 constant torch multiplies by."""
    return np.float32(d ** -0.5)


def fwht(x: np.ndarray) -> np.ndarray:
    """Orthonormal FWHT (reference hadamard.py:23-48)."""
    x = fwht_unscaled(x)
    return (x * fwht_scale(x.shape[-1])).astype(np.float32)


def rht(x: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """y = fwht(x * s)  (reference hadamard.py:70-90)."""
    return fwht(np.asarray(x, np.float32) * np.asarray(signs, np.float32))


def inverse_rht(y: np.ndarray, signs: np.ndarray) -> np.ndarray:
    """x = fwht(y) * s  (reference hadamard.py:93-100)."""
    return (fwht(y) * np.asarray(signs, np.float32)).astype(np.float32)


def sylvester(d: int) -> np.ndarray:
    """Unnormalised Sylvester Hadamard matrix H_d (float64)."""
    _check_pow2(d)
    h = np.ones((1, 1))
    while h.shape[0] < d:
        h = np.block([[h, h], [h, -h]])
    return h


# --------------------------------------------------------------------------
# Lloyd-Max codebook  (reference core/lloyd_max.py:24-88)
# --------------------------------------------------------------------------


def lloyd_max_codebook(dim: int, bits: int, max_iterations: int = 300,
                       num_grid_points: int = 50000):
    """Grid Lloyd-Max on the density (1 - z^2)^((d-3)/2) over [-6/sqrt d, 6/sqrt d].

    Returns ``(boundaries[2^b + 1], levels[2^b])`` in float64.
    """
    n = 1 << bits
    expo = (dim - 3) / 2.0
    sigma = 1.0 / math.sqrt(dim)
    lo = max(-1.0, -6.0 * sigma)
    hi = min(1.0, 6.0 * sigma)
    grid = np.linspace(lo, hi, num_grid_points)
    w = np.maximum(1.0 - grid ** 2, 0.0) ** expo
    w /= w.sum()
    bnd = np.interp(np.linspace(0, 1, n + 1), np.cumsum(w), grid)
    bnd[0] = lo
    bnd[-1] = hi
    lev = np.zeros(n)

    def centroids():
        for i in range(n):
            if i == n - 1:
                m = (grid >= bnd[i]) & (grid <= bnd[i + 1])
            else:
                m = (grid >= bnd[i]) & (grid < bnd[i + 1])
            ww = w[m]
            if ww.sum() > 0:
                lev[i] = np.average(grid[m], weights=ww)
            else:
                lev[i] = (bnd[i] + bnd[i + 1]) / 2.0

    centroids()
    for _ in range(max_iterations):
        for i in range(1, n):
            bnd[i] = (lev[i - 1] + lev[i]) / 2.0
        centroids()
    return bnd, lev


# --------------------------------------------------------------------------
# Quantise / pack  (reference core/lloyd_max.py:121-136, core/packing.py)
# --------------------------------------------------------------------------


def quantize(u: np.ndarray, boundaries: np.ndarray, bits: int) -> np.ndarray:
    """``clamp(bucketize(u, B, right=False) - 1, 0, 2^b - 1)`` as uint8.

    torch.bucketize(right=False) returns i with B[i-1] < u <= B[i], i.e. the
    number of boundaries strictly below u -- numpy's searchsorted(side='left').
    """
    b = np.asarray(boundaries, np.float32)
    idx = np.searchsorted(b, np.asarray(u, np.float32), side="left").astype(np.int64) - 1
    return np.clip(idx, 0, (1 << bits) - 1).astype(np.uint8)


def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    c = np.asarray(codes).astype(np.uint32)
    d = c.shape[-1]
    lead = c.shape[:-1]
    if bits == 4:
        v = c.reshape(*lead, d // 2, 2)
        return ((v[..., 1] << 4) | v[..., 0]).astype(np.uint8)
    if bits == 2:
        v = c.reshape(*lead, d // 4, 4)
        return (v[..., 0] | (v[..., 1] << 2) | (v[..., 2] << 4) | (v[..., 3] << 6)).astype(np.uint8)
    if bits == 3:
        v = c.reshape(*lead, d // 8, 8)
        w = np.zeros(v.shape[:-1], np.uint32)
        for k in range(8):
            w |= (v[..., k] & 7) << (3 * k)
        out = np.stack([w & 255, (w >> 8) & 255, (w >> 16) & 255], axis=-1)
        return out.reshape(*lead, d * 3 // 8).astype(np.uint8)
    if bits == 1:
        v = c.reshape(*lead, d // 8, 8)
        w = np.zeros(v.shape[:-1], np.uint32)
        for k in range(8):
            w |= (v[..., k] & 1) << k
        return w.astype(np.uint8)
    if bits == 8:
        return c.astype(np.uint8)
    raise ValueError(bits)


def unpack(packed: np.ndarray, bits: int, d: int) -> np.ndarray:
    p = np.asarray(packed).astype(np.uint32)
    lead = p.shape[:-1]
    if bits == 4:
        return np.stack([p & 15, p >> 4], axis=-1).reshape(*lead, d).astype(np.uint8)
    if bits == 2:
        return np.stack([(p >> s) & 3 for s in (0, 2, 4, 6)], axis=-1).reshape(*lead, d).astype(np.uint8)
    if bits == 3:
        g = p.reshape(*lead, d // 8, 3)
        w = g[..., 0] | (g[..., 1] << 8) | (g[..., 2] << 16)
        return np.stack([(w >> (3 * k)) & 7 for k in range(8)], axis=-1).reshape(*lead, d).astype(np.uint8)
    if bits == 1:
        return np.stack([(p >> k) & 1 for k in range(8)], axis=-1).reshape(*lead, d).astype(np.uint8)
    if bits == 8:
        return p.astype(np.uint8)
    raise ValueError(bits)


def packed_dim(d: int, bits: int) -> int:
    return (d * bits + 7) // 8


# --------------------------------------------------------------------------
# Library-format encode / decode  (reference core/quantizer.py:137-205)
# --------------------------------------------------------------------------


def l2norm_f32(y: np.ndarray) -> np.ndarray:
    """Per-vector Euclidean norm of float32 rows, correctly rounded to float32."""
    y64 = np.asarray(y, np.float64)
    return np.sqrt(np.sum(y64 * y64, axis=-1)).astype(np.float32)


def encode(x: np.ndarray, signs: np.ndarray, boundaries: np.ndarray, bits: int):
    """Returns ``(packed u8, norms f16, u f32, norms f32)``.

    ``u`` are the normalised rotated coordinates fed to the quantiser; the
    tests use them to identify codebook-boundary ties.
    """
    y = rht(np.asarray(x, np.float32), signs)
    n = l2norm_f32(y)
    u = (y / (n[..., None] + np.float32(1e-8))).astype(np.float32)
    codes = quantize(u, boundaries, bits)
    return pack(codes, bits), n.astype(np.float16), u, n


def decode(packed: np.ndarray, norms16: np.ndarray, levels: np.ndarray, signs: np.ndarray,
           bits: int, d: int) -> np.ndarray:
    codes = unpack(packed, bits, d)
    lev = np.asarray(levels, np.float32)[codes]
    r = (lev * np.asarray(norms16, np.float16).astype(np.float32)[..., None]).astype(np.float32)
    return inverse_rht(r, signs)


def tie_ulps(u: np.ndarray, cuts: np.ndarray, d: int) -> np.ndarray:
    """Distance of u to the nearest of `cuts` (float32 values: interior
    boundaries or midpoints), in float32 ulps of max(|cut|, d**-0.5): the
    rounding of the rotated coordinate (a sum of d terms of size ~d**-0.5 in
    normalised units) is measured against that scale, also at a cut near 0."""
    c = np.asarray(cuts, np.float32)
    scale = np.spacing(np.maximum(np.abs(c), np.float32(d ** -0.5)).astype(np.float32)).astype(np.float64)
    uu = np.asarray(u, np.float64)[..., None]
    return np.min(np.abs(uu - c.astype(np.float64)) / scale, axis=-1)


def boundary_distance(u: np.ndarray, boundaries: np.ndarray) -> np.ndarray:
    """|u - nearest interior boundary| (float64), for tie accounting."""
    b = np.asarray(boundaries, np.float32).astype(np.float64)[1:-1]
    uu = np.asarray(u, np.float64)[..., None]
    return np.min(np.abs(uu - b), axis=-1)


# --------------------------------------------------------------------------
# Dense library-format decode attention (float64)
# reference vllm_plugin/attention_impl.py:431-521, kernels/triton_flash_decode.py
# --------------------------------------------------------------------------


def dense_decode_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, seq_lens, scale: float):
    """q [B, Hq, d]; k, v [B, Hkv, S, d] (already decoded); returns [B, Hq, d] float64.

    Positions >= seq_lens[b] are masked (reference attention_impl.py:492-498).
    GQA: q-head h reads kv-head h // (Hq // Hkv) (reference triton_flash_decode.py:71-75).
    """
    q = np.asarray(q, np.float64)
    B, Hq, d = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    out = np.zeros((B, Hq, d))
    for b in range(B):
        L = int(seq_lens[b])
        for h in range(Hq):
            kk = np.asarray(k[b, h // g, :L], np.float64)
            vv = np.asarray(v[b, h // g, :L], np.float64)
            s = kk @ q[b, h] * scale
            if L == 0:
                continue
            s = s - s.max()
            p = np.exp(s)
            out[b, h] = (p / p.sum()) @ vv
    return out


def lse_merge(parts_o: np.ndarray, parts_lse: np.ndarray):
    """Log-sum-exp merge of split results (vLLM stage 2 semantics).

    parts_o [..., S, d], parts_lse [..., S]; splits with lse = -inf are dropped.
    """
    m = np.max(parts_lse, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    w = np.exp(parts_lse - m)
    den = w.sum(-1)
    o = (w[..., None] * parts_o).sum(-2) / np.where(den > 0, den, 1.0)[..., None]
    return o, (m[..., 0] + np.log(np.where(den > 0, den, 1.0)))


# --------------------------------------------------------------------------
# Page layout reader (checker for the paged store of fused_turboquant.paged)
# --------------------------------------------------------------------------


def paged_unpack(cache: np.ndarray, d: int, bk: int, bv: int):
    """Read a paged library-format cache uint8[nb, Hkv, nsub, sub] back into
    per-token arrays: K codes / V codes [nb, Hkv, page, d] (uint8) and K / V
    norms [nb, Hkv, page] (float16).

    Sub-block layout (16 tokens): K codes [16][d*bk/8] per-token packed;
    V codes [64 chunks][d*bv/32] where chunk c = 16*q + r holds, for d-block
    b, the codes of tokens 4q+i (i = 0..3) at d = 16b + r, bit (4b + i)*bv;
    then K norms fp16[16], V norms fp16[16].
    """
    nb, hkv, nsub, sub = cache.shape
    ktok = d * bk // 8
    ksec = 16 * ktok
    vlane = d * bv // 32
    vsec = 64 * vlane
    assert sub == ksec + vsec + 64
    c = cache.reshape(nb, hkv, nsub, sub)
    kc = unpack(c[..., :ksec].reshape(nb, hkv, nsub, 16, ktok), bk, d)
    vbytes = c[..., ksec:ksec + vsec].reshape(nb, hkv, nsub, 64, vlane)
    bits = np.unpackbits(vbytes, axis=-1, bitorder="little").astype(np.uint32)
    vc = np.zeros((nb, hkv, nsub, 16, d), np.uint8)
    for q in range(4):
        for r in range(16):
            ch = bits[..., 16 * q + r, :]
            for b in range(d // 16):
                for i in range(4):
                    p = (4 * b + i) * bv
                    code = np.zeros(ch.shape[:-1], np.uint32)
                    for k in range(bv):
                        code |= ch[..., p + k] << k
                    vc[..., 4 * q + i, 16 * b + r] = code
    kn = c[..., ksec + vsec:ksec + vsec + 32].copy().view(np.float16).reshape(nb, hkv, nsub, 16)
    vn = c[..., ksec + vsec + 32:].copy().view(np.float16).reshape(nb, hkv, nsub, 16)
    page = nsub * 16
    return (kc.reshape(nb, hkv, page, d), vc.reshape(nb, hkv, page, d),
            kn.reshape(nb, hkv, page), vn.reshape(nb, hkv, page))


# --------------------------------------------------------------------------
# vLLM v1 TURBOQUANT slot format
# store:  reference vllm_plugin/triton_inkernel_store.py:38-440 (_fused_store_rht
#         + _bucketize_pack_norm_v_store), v1_backend.py:712-749 (v_rotate)
# decode: reference vllm_plugin/triton_decode_offset.py:42-442 (stage 1),
#         v1_backend.py:975-1093 (stage 2 merge, un-rotation, output cast)
# geometry: reference boundary_tq_config.py:66-81, v1_backend.py:171-220
# --------------------------------------------------------------------------


def v1_geometry(d: int, kb: int, vb: int, key_fp8: bool = False) -> dict:
    """Byte offsets inside one (token, kv head) slot.

    ``[K codes: mse][K norm f16][V codes: vdb][V scale f16][V zero f16][pad]``;
    key_packed_size = mse + 2 (boundary_tq_config.py:66-75), or d with fp8
    keys and no norm (:66-73); value data bytes = ceil(d * vb / 8), d at 8 bits
    (:77-81); raw = kps + vdb + 4, slot = next power of 2 (v1_backend.py:206-209,
    boundary protection off).
    """
    mse = d if key_fp8 else -(-d * kb // 8)
    kps = mse if key_fp8 else mse + 2
    vdb = d if vb == 8 else -(-d * vb // 8)
    raw = kps + vdb + 4
    slot = 1 << (raw - 1).bit_length()
    return dict(mse=mse, kps=kps, vdb=vdb, raw=raw, slot=slot)


def v1_midpoints(centroids: np.ndarray) -> np.ndarray:
    """Sorted centroids -> float32 midpoints (c[i] + c[i+1]) / 2
    (reference rotation/matrix.py:34-42)."""
    c = np.sort(np.asarray(centroids, np.float32))
    return ((c[:-1] + c[1:]) / np.float32(2)).astype(np.float32)


def v1_quantize_k(y: np.ndarray, midpoints: np.ndarray) -> np.ndarray:
    """Binary search over the midpoints with ``y >= m`` going up
    (triton_inkernel_store.py:91-100): the number of midpoints <= y."""
    m = np.asarray(midpoints, np.float32)
    return np.searchsorted(m, np.asarray(y, np.float32), side="right").astype(np.uint8)


def v1_blockdiag_rotate(x: np.ndarray, coeffs: np.ndarray, B: int) -> np.ndarray:
    """x M for a block-diagonal M given by coeffs[j][e] = M[(e // B) B + j][e]:
    y[e] = fma(x_{B-1}, c_{B-1}, ... fma(x_1, c_1, x_0 c_0)) in float32 with
    x_j = x[(e // B) B + j] (reference _fused_store_block_diag,
    triton_inkernel_store.py:727-742).  Each fused step is the exact product
    plus the sum formed in float64, then rounded to float32."""
    x = np.asarray(x, np.float32)
    c = np.asarray(coeffs, np.float32)
    d = x.shape[-1]
    e = np.arange(d)
    y = None
    for j in range(B):
        src = (e // B) * B + j
        ok = src < d
        xp = np.where(ok, x[..., np.minimum(src, d - 1)], np.float32(0)).astype(np.float64)
        prod = xp * c[j].astype(np.float64)
        y = prod.astype(np.float32) if j == 0 else (prod + y.astype(np.float64)).astype(np.float32)
    return y


def v1_k_rotate(k: np.ndarray, rotation=None, blockdiag=None):
    """K path before the quantiser (triton_inkernel_store.py:406-430):
    norm = sqrt(sum k^2 + 1e-16); x = k / (norm + 1e-8); y = H x / sqrt(d)
    (Sylvester butterflies, no random signs).  Returns (y f32, norm f32)."""
    k = np.asarray(k, np.float32)
    d = k.shape[-1]
    k64 = k.astype(np.float64)
    norm = np.sqrt(np.sum(k64 * k64, axis=-1) + 1e-16).astype(np.float32)
    x = (k / (norm[..., None] + np.float32(1e-8))).astype(np.float32)
    if blockdiag is not None:  # k * (1 / (norm + 1e-8)), then the block products (:718-742)
        inv = (np.float32(1.0) / (norm + np.float32(1e-8))).astype(np.float32)
        x = (k * inv[..., None]).astype(np.float32)
        y = v1_blockdiag_rotate(x, *blockdiag)
    elif rotation is None:
        y = (fwht_unscaled(x) * fwht_scale(d)).astype(np.float32)
    else:  # a matrix strategy: x M (MatrixRotationStrategy.rotate_for_store, rotation/matrix.py:44-45)
        y = (x.astype(np.float64) @ np.asarray(rotation, np.float64)).astype(np.float32)
    return y, norm


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    """float32 -> fp8 e4m3fn bytes (bias 7, 3 mantissa bits, no infinities,
    0x7f / 0xff NaN), rounding to nearest even and saturating at +-448 --
    the reference's ``y.to(tl.float8e4nv)`` of the fp8-key store
    (triton_inkernel_store.py:76-82), whose out-of-range behaviour
    (saturation) is parity unpinned: torch's own e4m3fn conversion gives NaN
    there, and the two agree below 464.  Each byte is the encoding whose value
    is nearest in float64 (ties to the even mantissa)."""
    x = np.asarray(x, np.float32)
    codes = np.arange(256, dtype=np.uint32)
    vals = e4m3_to_f32(codes).astype(np.float64)
    pos = codes[:127][np.argsort(vals[:127])]  # 0x00 .. 0x7e: +0 .. 448, increasing
    pv = vals[pos]
    a = np.abs(x.astype(np.float64))
    i = np.clip(np.searchsorted(pv, a, side="left"), 1, pos.size - 1)
    lo, hi = pv[i - 1], pv[i]
    take_hi = (a - lo > hi - a) | ((a - lo == hi - a) & ((pos[i] & 1) == 0))
    out = np.where(take_hi, pos[i], pos[i - 1])
    out = np.where(a >= 448.0, 0x7E, out)  # saturate (infinities included)
    out = np.where(np.isnan(x), 0x7F, out)
    sign = (x.view(np.uint32) >> 24) & 0x80
    return (out | sign).astype(np.uint8)


def e4m3_to_f32(b: np.ndarray) -> np.ndarray:
    """fp8 e4m3fn bytes -> float32: (-1)^s 2^(e-7) (1 + m/8) for e > 0,
    (-1)^s m 2^-9 for e = 0, NaN for 0x7f / 0xff."""
    b = np.asarray(b).astype(np.uint32)
    e = (b >> 3) & 15
    m = b & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e.astype(np.float64) - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(b & 0x80, -v, v).astype(np.float32)


def v1_quantize_v(v: np.ndarray, vb: int):
    """Per-vector uniform min/max quantiser (triton_inkernel_store.py:202-330).

    Returns (codes u8, scale f32, min f32, t f32) where t = (v - mn) / sc + 0.5
    is the value truncated to the code (kept for tie accounting).
    """
    v = np.asarray(v, np.float32)
    mn = v.min(axis=-1)
    mx = v.max(axis=-1)
    top = (1 << vb) - 1
    if vb == 1:
        sc = (mx - mn).astype(np.float32)
    else:
        sc = ((mx - mn) / np.float32(top)).astype(np.float32)
    sc = np.where(sc > np.float32(1e-8), sc, np.float32(1e-8)).astype(np.float32)
    t = (((v - mn[..., None]).astype(np.float32) / sc[..., None]).astype(np.float32) + np.float32(0.5)).astype(np.float32)
    q = np.clip(np.trunc(t), 0, top).astype(np.uint8)
    return q, sc, mn, t


def v1_dense_rotation(d: int, rotation=None, blockdiag=None) -> np.ndarray:
    """The float32 d x d matrix M of the layer's rotation (``x @ M`` is the
    forward rotation): Sylvester H / sqrt(d) for ``rht`` (reference
    rotation/hadamard.py:28-34, a float32 tensor divided by the Python float
    sqrt(d)), the caller's matrix, or the block-diagonal matrix whose
    coefficients coeffs[j][e] = M[(e // B) B + j][e] are given
    (rotation/matrix.py:104-148)."""
    if blockdiag is not None:
        coeffs, B = blockdiag
        c = np.asarray(coeffs, np.float32)
        m = np.zeros((d, d), np.float32)
        for e in range(d):
            for j in range(B):
                r = (e // B) * B + j
                if r < d:
                    m[r, e] = c[j][e]
        return m
    if rotation is not None:
        return np.asarray(rotation, np.float32)
    return (sylvester(d).astype(np.float32) / np.float32(math.sqrt(d))).astype(np.float32)


def v1_rotate_value(value: np.ndarray, M: np.ndarray) -> np.ndarray:
    """V pre-rotation of ``v_rotate`` / ``V_LLOYD_MAX`` (reference
    v1_backend.py:736-740): ``einsum('nhd,de->nhe', value.float(), M)`` with
    the layer's float32 matrix M, cast back to the value dtype afterwards.
    The einsum is a float32 GEMM whose summation order is the library's; the
    value every such order approximates is the product formed here in
    float64 (bf16/fp16/fp32 inputs times float32 entries: each product exact,
    the sum within ~2^-50 relative).  How far a float32 order may stray from
    it is bounded in ``v1_v_tie_vectors``."""
    return np.asarray(value, np.float32).astype(np.float64) @ np.asarray(M, np.float32).astype(np.float64)


# Spread allowed between float32 evaluations of the V pre-rotation, in units
# of 2^-24 * rms of the rotated vector.  Measured on N(0,1) bf16 vectors with
# 2% x8 outliers (d = 64 / 128 / 256): the Sylvester butterflies stay within
# 5.2, an sgemm and a sequential float32 dot product within 43 (d = 128, where
# 1/sqrt(d) is not a power of two and each product rounds).
V_TIE_UNITS = 64.0


def v1_v_tie_vectors(vr: np.ndarray, dtype: str, vb: int, v_lloyd_max: bool = False,
                     units: float = V_TIE_UNITS) -> np.ndarray:
    """Boolean [...] mask of the vectors whose stored V bytes can depend on
    the float32 summation order of the pre-rotation: with every rotated
    element moved anywhere within +-tol (tol = units * 2^-24 * rms of the
    vector) of its exact value ``vr`` (float64, ``v1_rotate_value``), a
    vector is flagged if its stored fields can take more than one value:

    * the rounded element takes two values (it sits within tol of a rounding
      boundary of the value dtype; for float32 every element moves) and that
      changes its code, the minimum or the maximum;
    * uniform codes: the range of (v - min) / scale + 0.5 over the box
      straddles an integer, or the fp16 scale or minimum straddles an fp16
      rounding boundary;
    * Lloyd-Max codes (``v_lloyd_max``, 4-bit V): any element takes two
      values (the norm and every code depend on all of them).

    Interval arithmetic on monotone float32 formulas, so the mask is a
    superset of the vectors any float32 order can change."""
    vr = np.asarray(vr, np.float64)
    rms = np.sqrt(np.mean(vr * vr, axis=-1, keepdims=True))
    tol = units * 2.0 ** -24 * rms
    lo = v1_round_dtype((vr - tol).astype(np.float32), dtype)
    hi = v1_round_dtype((vr + tol).astype(np.float32), dtype)
    if v_lloyd_max and vb == 4:
        # codes and the fp16 norm both depend on every element: any element
        # with two candidate values flags the vector
        return np.any(lo != hi, axis=-1)
    top = (1 << vb) - 1
    mn_lo, mn_hi = lo.min(axis=-1), hi.min(axis=-1)
    mx_lo, mx_hi = lo.max(axis=-1), hi.max(axis=-1)

    def _scale(mx, mn):
        s = (mx - mn).astype(np.float32) if vb == 1 else ((mx - mn) / np.float32(top)).astype(np.float32)
        return np.where(s > np.float32(1e-8), s, np.float32(1e-8)).astype(np.float32)

    sc_min, sc_max = _scale(mx_lo, mn_hi), _scale(mx_hi, mn_lo)
    flag = (mn_lo.astype(np.float16) != mn_hi.astype(np.float16)) | \
           (sc_min.astype(np.float16) != sc_max.astype(np.float16))

    def _t(v, mn, sc):
        return (((v - mn[..., None]).astype(np.float32) / sc[..., None]).astype(np.float32)
                + np.float32(0.5)).astype(np.float32)

    # (v - mn) / sc grows with v and falls with mn; where v - mn >= 0 it falls
    # with sc.  The upper corner (hi, mn_lo, sc_min) always has hi - mn_lo >= 0;
    # a lower corner with lo - mn_hi < 0 gives t < 0.5, code 0, the least code
    t_lo = _t(lo, mn_hi, sc_max)
    t_hi = _t(hi, mn_lo, sc_min)
    c_lo = np.clip(np.floor(np.maximum(t_lo, 0)), 0, top)
    c_hi = np.clip(np.floor(np.maximum(t_hi, 0)), 0, top)
    return flag | np.any(c_lo != c_hi, axis=-1)


def v1_round_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 -> value dtype -> float32 (round to nearest even)."""
    x = np.asarray(x, np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        nan = np.isnan(x)
        out = r.astype(np.uint32).view(np.float32)
        return np.where(nan, x, out).astype(np.float32)
    raise ValueError(dtype)


def v1_quantize_v_lloyd(v: np.ndarray, midpoints: np.ndarray):
    """Lloyd-Max V codes (TURBOQUANT_V_LLOYD_MAX, 4-bit V;
    triton_inkernel_store.py:159-200): norm = sqrt(sum v^2 + 1e-16),
    u = v / (norm + 1e-8), code = the K midpoint search on u (``>=`` going up).
    Returns (codes u8, norm f32, u f32)."""
    v = np.asarray(v, np.float32)
    v64 = v.astype(np.float64)
    norm = np.sqrt(np.sum(v64 * v64, axis=-1) + 1e-16).astype(np.float32)
    u = (v / (norm[..., None] + np.float32(1e-8))).astype(np.float32)
    return v1_quantize_k(u, midpoints), norm, u


def v1_store(key: np.ndarray, value: np.ndarray, slot_mapping: np.ndarray, kv_cache: np.ndarray,
             midpoints: np.ndarray, kb: int, vb: int, v_rotate: bool = False,
             value_dtype: str = "f32", v_lloyd_max: bool = False, rotation=None, blockdiag=None,
             key_fp8: bool = False):
    """Write [N, H, d] float32 K/V (already converted from their dtype) into
    ``kv_cache`` uint8[nb, bs, H, slot] in place.  Negative slots are skipped
    (triton_inkernel_store.py:394-395).  With ``v_rotate`` V is first rotated
    by the layer's dense M (``v1_rotate_value``: H/sqrt(d), the caller's
    matrix, or the block-diagonal one) and rounded back to the value dtype
    (v1_backend.py:736-740); ``vrot`` in the result is that product before
    the rounding, for ``v1_v_tie_vectors``.
    With ``v_lloyd_max`` and 4-bit V, V takes Lloyd-Max codes against the K
    midpoints, its norm goes in the scale field and the min field is 0
    (triton_inkernel_store.py:159-200); other V widths keep the uniform codes.
    ``blockdiag`` = (coeffs [B, d], B): a block-diagonal strategy, K and the
    rotated V formed by v1_blockdiag_rotate.  With ``key_fp8`` (key bits 8) K
    is stored as fp8 e4m3fn bytes of y * norm and no norm
    (triton_inkernel_store.py:59-83).

    Returns a dict of per-(token, head) intermediates for tie accounting.
    """
    key = np.asarray(key, np.float32)
    value = np.asarray(value, np.float32)
    N, H, d = key.shape
    nb, bs, Hc, slot = kv_cache.shape
    assert Hc == H
    g = v1_geometry(d, kb, vb, key_fp8)
    y, norm = v1_k_rotate(key, rotation, blockdiag)
    if key_fp8:
        kcodes = f32_to_e4m3((y * norm[..., None]).astype(np.float32))
    else:
        kcodes = v1_quantize_k(y, midpoints)
    vr = None
    if v_rotate:
        vr = v1_rotate_value(value, v1_dense_rotation(d, rotation, blockdiag))
        value = v1_round_dtype(vr.astype(np.float32), value_dtype)
    if v_lloyd_max and vb == 4:
        vq, sc, t = v1_quantize_v_lloyd(value, midpoints)
        mn = np.zeros_like(sc)
    else:
        vq, sc, mn, t = v1_quantize_v(value, vb)
    kp = kcodes if key_fp8 else pack(kcodes, kb)
    vp = pack(vq, vb)
    n16 = norm.astype(np.float16).view(np.uint8).reshape(N, H, 2)
    sc16 = sc.astype(np.float16).view(np.uint8).reshape(N, H, 2)
    mn16 = mn.astype(np.float16).view(np.uint8).reshape(N, H, 2)
    for i in range(N):
        s = int(slot_mapping[i])
        if s < 0:
            continue
        blk, off = divmod(s, bs)
        row = kv_cache[blk, off]
        row[:, 0:g["mse"]] = kp[i]
        if not key_fp8:
            row[:, g["mse"]:g["kps"]] = n16[i]
        row[:, g["kps"]:g["kps"] + g["vdb"]] = vp[i]
        row[:, g["kps"] + g["vdb"]:g["kps"] + g["vdb"] + 2] = sc16[i]
        row[:, g["kps"] + g["vdb"] + 2:g["raw"]] = mn16[i]
    return dict(y=y, norm=norm, kcodes=kcodes, vcodes=vq, vscale=sc, vmin=mn, vt=t, value=value, vrot=vr)


def v1_unpack(kv_cache: np.ndarray, d: int, kb: int, vb: int, key_fp8: bool = False):
    """uint8[nb, bs, H, slot] -> (K codes, K norm f16, V codes, V scale f16,
    V zero f16), codes [nb, bs, H, d].  With ``key_fp8`` the K "codes" are the
    fp8 bytes and the K norm is None."""
    g = v1_geometry(d, kb, vb, key_fp8)
    c = np.asarray(kv_cache)
    if key_fp8:
        kc = c[..., :d].copy()
        kn = None
    else:
        kc = unpack(c[..., :g["mse"]], kb, d)
        kn = c[..., g["mse"]:g["kps"]].copy().view(np.float16)[..., 0]
    vc = unpack(c[..., g["kps"]:g["kps"] + g["vdb"]], vb, d)
    sc = c[..., g["kps"] + g["vdb"]:g["kps"] + g["vdb"] + 2].copy().view(np.float16)[..., 0]
    zr = c[..., g["kps"] + g["vdb"] + 2:g["raw"]].copy().view(np.float16)[..., 0]
    return kc, kn, vc, sc, zr


def v1_dequant(kv_cache: np.ndarray, d: int, kb: int, vb: int, centroids: np.ndarray,
               norm_correction: bool = True, v_lloyd_max: bool = False, key_fp8: bool = False):
    """Per-slot reconstructions in the rotated domain (float64):
    K^ = ||k||_16 * c / sqrt(sum c^2 + 1e-16)  (triton_decode_offset.py:210-242),
    V^ = q * scale_16 + zero_16               (:256-428), or with
    ``v_lloyd_max`` and 4-bit V V^ = ||v||_16 * c_v / sqrt(sum c_v^2 + 1e-16)
    (:399-419; the scale field holds ||v||, the K centroids are shared).
    fp8 keys: K^ = the fp8 values themselves (:174-192)."""
    kc, kn, vc, sc, zr = v1_unpack(kv_cache, d, kb, vb, key_fp8)
    cs = np.sort(np.asarray(centroids, np.float32)).astype(np.float64) if centroids is not None else None
    if key_fp8:
        k_hat = e4m3_to_f32(kc).astype(np.float64)
    else:
        c = cs[kc]
        if norm_correction:
            c = c / np.sqrt(np.sum(c * c, axis=-1, keepdims=True) + 1e-16)
        k_hat = c * kn.astype(np.float64)[..., None]
    if v_lloyd_max and vb == 4:
        cv = cs[np.minimum(vc, cs.size - 1)]
        if norm_correction:
            cv = cv / np.sqrt(np.sum(cv * cv, axis=-1, keepdims=True) + 1e-16)
        return k_hat, cv * sc.astype(np.float64)[..., None]
    v_hat = vc.astype(np.float64) * sc.astype(np.float64)[..., None] + zr.astype(np.float64)[..., None]
    return k_hat, v_hat


def v1_decode_attention(q: np.ndarray, kv_cache: np.ndarray, block_table: np.ndarray,
                        seq_lens: np.ndarray, centroids: np.ndarray, kb: int, vb: int,
                        scale: float, kv_start=None, v_rotate: bool = False,
                        norm_correction: bool = True, v_lloyd_max: bool = False,
                        rotation=None, key_fp8: bool = False):
    """Decode attention over the v1 slot cache, float64.

    q [B, Hq, d] (float32 values of the query); q_rot = q @ M with
    M = H / sqrt(d) (v1_backend.py:1004, rotation/matrix.py:44-48).  Positions
    [kv_start[b], seq_lens[b]) of sequence b are attended
    (triton_decode_offset.py:104-106); GQA head h reads kv head h // (Hq/Hkv).
    Output = softmax(s) . V^, then o @ M^T when v_rotate (v1_backend.py:1086-1092).
    Rows with no positions return zeros (this library's convention).
    """
    q = np.asarray(q, np.float64)
    B, Hq, d = q.shape
    nb, bs, Hkv, slot = kv_cache.shape
    G = Hq // Hkv
    M = sylvester(d) / math.sqrt(d) if rotation is None else np.asarray(rotation, np.float64)
    q_rot = q @ M
    k_hat, v_hat = v1_dequant(kv_cache, d, kb, vb, centroids, norm_correction, v_lloyd_max, key_fp8)
    out = np.zeros((B, Hq, d))
    for b in range(B):
        L = int(seq_lens[b])
        s0 = 0 if kv_start is None else int(kv_start[b])
        if L <= s0:
            continue
        pos = np.arange(s0, L)
        blk = np.asarray(block_table[b])[pos // bs]
        off = pos % bs
        for h in range(Hq):
            kk = k_hat[blk, off, h // G]
            vv = v_hat[blk, off, h // G]
            s = kk @ q_rot[b, h] * scale
            s = s - s.max()
            p = np.exp(s)
            o = (p / p.sum()) @ vv
            out[b, h] = (o @ M.T) if v_rotate else o
    return out


def v1_hybrid_decode_attention(q: np.ndarray, prefix_k: np.ndarray, prefix_v: np.ndarray, prefix_len: int,
                               kv_cache: np.ndarray, block_table: np.ndarray, seq_lens: np.ndarray,
                               centroids: np.ndarray, kb: int, vb: int, scale: float,
                               v_rotate: bool = False, norm_correction: bool = True):
    """Deferred-prefill decode, float64 (reference v1_backend.py:1095-1277).

    prefix_k / prefix_v [P_cap, Hkv, d]: the fp16 prefix rows (values as
    stored).  Sequence 0 attends prefix rows [0, prefix_len) (the reference's
    cu_seqlens_k = [0, P, P, ...] give the other sequences none) plus the
    quantised slot positions [prefix_len, seq_lens[0]); sequence b > 0 attends
    only its positions [prefix_len, seq_lens[b]).  Prefix scores are q . k in
    the original domain, slot scores q M . K^ in the rotated one (equal for an
    orthogonal M); rotated V^ rows are taken back by M^T when v_rotate.  One
    softmax over all of them -- what the reference's LSE merge of the two
    phases computes."""
    q = np.asarray(q, np.float64)
    B, Hq, d = q.shape
    nb, bs, Hkv, slot = kv_cache.shape
    G = Hq // Hkv
    M = sylvester(d) / math.sqrt(d)
    q_rot = q @ M
    k_hat, v_hat = v1_dequant(kv_cache, d, kb, vb, centroids, norm_correction)
    pk = np.asarray(prefix_k, np.float64)
    pv = np.asarray(prefix_v, np.float64)
    out = np.zeros((B, Hq, d))
    for b in range(B):
        P = prefix_len if b == 0 else 0
        L = int(seq_lens[b])
        pos = np.arange(prefix_len, L) if L > prefix_len else np.arange(0)
        blk = np.asarray(block_table[b])[pos // bs]
        off = pos % bs
        for h in range(Hq):
            kv = h // G
            s_p = pk[:P, kv] @ q[b, h] * scale
            s_q = k_hat[blk, off, kv] @ q_rot[b, h] * scale
            vq = v_hat[blk, off, kv]
            if v_rotate:
                vq = vq @ M.T
            s = np.concatenate([s_p, s_q])
            if s.size == 0:
                continue
            w = np.exp(s - s.max())
            out[b, h] = (w / w.sum()) @ np.concatenate([pv[:P, kv], vq])
    return out


# --------------------------------------------------------------------------
# raw fp16 slots of the boundary layers
#   store:  vllm_plugin/v1_backend.py:1449-1505 (_store_raw_kv)
#   decode: vllm_plugin/triton_boundary_attn.py:28-219 (one program per
#           (batch, q head), online softmax over the block-table positions)
# --------------------------------------------------------------------------


def raw_store(key: np.ndarray, value: np.ndarray, slot_mapping: np.ndarray,
              kv_cache: np.ndarray) -> None:
    """Write key/value [n, Hkv, d] as float16 into kv_cache
    uint8[nb, bs, Hkv, slot] at [K fp16 | V fp16]; negative slots skipped."""
    n, hkv, d = key.shape
    nb, bs = kv_cache.shape[0], kv_cache.shape[1]
    with np.errstate(over="ignore"):  # fp16 overflow -> inf, as .to(float16) does
        k16 = np.asarray(key, np.float32).astype(np.float16).view(np.uint8).reshape(n, hkv, 2 * d)
        v16 = np.asarray(value, np.float32).astype(np.float16).view(np.uint8).reshape(n, hkv, 2 * d)
    for i in range(n):
        s = int(slot_mapping[i])
        if s < 0 or s // bs >= nb:
            continue
        kv_cache[s // bs, s % bs, :, : 2 * d] = k16[i]
        kv_cache[s // bs, s % bs, :, 2 * d: 4 * d] = v16[i]


def raw_unpack(kv_cache: np.ndarray, d: int):
    """(K, V) float64 [nb, bs, Hkv, d] from raw slots."""
    nb, bs, hkv, slot = kv_cache.shape
    c = np.ascontiguousarray(kv_cache[..., : 4 * d])
    k = c[..., : 2 * d].copy().view(np.float16).astype(np.float64)
    v = c[..., 2 * d: 4 * d].copy().view(np.float16).astype(np.float64)
    return k, v


def raw_decode_attention(q: np.ndarray, kv_cache: np.ndarray, block_table: np.ndarray,
                         seq_lens: np.ndarray, scale: float, kv_start=None) -> np.ndarray:
    """float64 softmax(q . K^T * scale) . V over positions [kv_start[b],
    seq_lens[b]) of block-table row b; kv head h // (Hq/Hkv); empty rows 0."""
    q = np.asarray(q, np.float64)
    B, Hq, d = q.shape
    nb, bs, Hkv, slot = kv_cache.shape
    G = Hq // Hkv
    k_all, v_all = raw_unpack(kv_cache, d)
    out = np.zeros((B, Hq, d))
    for b in range(B):
        L = int(seq_lens[b])
        s0 = 0 if kv_start is None else int(kv_start[b])
        if L <= s0:
            continue
        pos = np.arange(s0, L)
        blk = np.asarray(block_table[b])[pos // bs]
        off = pos % bs
        for h in range(Hq):
            kk = k_all[blk, off, h // G]
            vv = v_all[blk, off, h // G]
            s = kk @ q[b, h] * scale
            s = s - s.max()
            p = np.exp(s)
            out[b, h] = (p / p.sum()) @ vv
    return out
