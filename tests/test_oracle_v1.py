"""The v1 TURBOQUANT slot-format oracle pinned against the reference's stated
byte counts and against closed forms.

vLLM (``get_centroids``, the stage-2 merge kernel, ``TurboQuantConfig``) is not
in the reference tree, so nothing here compares against vLLM outputs; each
check below is one a plausible restatement mistake would fail.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O


@pytest.mark.parametrize("bits,raw", [(2, 70), (3, 102), (4, 134), (8, 262)])
def test_geometry_matches_reference_slot_bytes(bits, raw):
    # reference README.md:247-252: bytes used per slot at head_dim 128
    g = O.v1_geometry(128, bits, bits)
    assert g["raw"] == raw
    assert g["kps"] == 128 * bits // 8 + 2


def test_geometry_mixed_bits():
    # K4V2: K region 66, V region 32 + 4 (reference boundary_tq_config.py:66-81)
    g = O.v1_geometry(128, 4, 2)
    assert (g["mse"], g["kps"], g["vdb"], g["raw"], g["slot"]) == (64, 66, 32, 102, 128)
    assert O.v1_geometry(128, 4, 4)["slot"] == 256


def test_quantize_k_is_nearest_centroid_with_upper_ties():
    c = np.sort(np.random.default_rng(0).standard_normal(16).astype(np.float32) * 0.1)
    m = O.v1_midpoints(c)
    y = np.random.default_rng(1).standard_normal(4000).astype(np.float32) * 0.15
    y = np.concatenate([y, m, np.nextafter(m, -np.inf, dtype=np.float32)])
    got = O.v1_quantize_k(y, m)
    # brute force: nearest centroid; at an exact midpoint the upper one
    dist = np.abs(y[:, None].astype(np.float64) - c[None, :].astype(np.float64))
    mids64 = m.astype(np.float64)
    want = np.argmin(dist, axis=1)
    on_mid = np.isin(y.astype(np.float64), mids64)
    idx_mid = np.searchsorted(mids64, y.astype(np.float64))
    want = np.where(on_mid, idx_mid + 1, want)
    # away from midpoints the float32 midpoint rounding cannot move the answer
    assert np.array_equal(got, want)
    # exact midpoints go up (the reference's `y >= mid` branch)
    assert np.array_equal(O.v1_quantize_k(m, m), np.arange(1, 16))


def test_midpoints_are_float32_half_sums():
    c = np.array([-0.3, -0.1, 0.1, 0.3], np.float32)
    assert np.array_equal(O.v1_midpoints(c[::-1]), np.array([-0.2, 0.0, 0.2], np.float32))


@pytest.mark.parametrize("d", [64, 128, 256])
def test_k_rotate_is_normalised_sylvester(d):
    rng = np.random.default_rng(d)
    k = rng.standard_normal((7, d)).astype(np.float32) * 3
    y, n = O.v1_k_rotate(k)
    want = (k.astype(np.float64) / np.linalg.norm(k, axis=-1, keepdims=True)) @ O.sylvester(d).T / math.sqrt(d)
    assert np.allclose(y, want, atol=2e-6)
    assert np.allclose(n, np.linalg.norm(k.astype(np.float64), axis=-1), rtol=1e-6)
    # no random signs: the first coordinate is the scaled sum
    assert np.allclose(y[:, 0], want[:, 0], atol=2e-6)


@pytest.mark.parametrize("vb", [1, 2, 3, 4, 8])
def test_quantize_v_error_bound_and_endpoints(vb):
    rng = np.random.default_rng(vb)
    v = rng.standard_normal((50, 128)).astype(np.float32)
    q, sc, mn, _ = O.v1_quantize_v(v, vb)
    top = (1 << vb) - 1
    rec = q.astype(np.float64) * sc[:, None] + mn[:, None]
    assert np.all(np.abs(rec - v) <= sc[:, None] * 0.5 * (1 + 1e-5) + 1e-7)
    assert np.array_equal(q[np.arange(50), v.argmin(-1)], np.zeros(50))
    assert np.array_equal(q[np.arange(50), v.argmax(-1)], np.full(50, top))
    want_sc = (v.max(-1) - v.min(-1)) / (np.float32(top) if vb > 1 else np.float32(1))
    assert np.array_equal(sc, want_sc.astype(np.float32))


def test_quantize_v_constant_vector_uses_floor_scale():
    q, sc, mn, _ = O.v1_quantize_v(np.full((1, 64), 2.5, np.float32), 3)
    assert sc[0] == np.float32(1e-8) and mn[0] == np.float32(2.5) and not q.any()


def test_store_roundtrip_and_skip():
    rng = np.random.default_rng(5)
    N, H, d, kb, vb = 9, 2, 128, 4, 2
    g = O.v1_geometry(d, kb, vb)
    cache = np.full((3, 4, H, 256), 0xAB, np.uint8)
    k = rng.standard_normal((N, H, d)).astype(np.float32)
    v = rng.standard_normal((N, H, d)).astype(np.float32)
    c = O.lloyd_max_codebook(d, kb)[1].astype(np.float32)
    slots = np.array([0, 5, -1, 11, 2, 3, 7, 6, 1])
    st = O.v1_store(k, v, slots, cache, O.v1_midpoints(c), kb, vb)
    kc, kn, vc, sc, zr = O.v1_unpack(cache, d, kb, vb)
    for i, s in enumerate(slots):
        if s < 0:
            continue
        b, o = divmod(int(s), 4)
        assert np.array_equal(kc[b, o], st["kcodes"][i])
        assert np.array_equal(vc[b, o], st["vcodes"][i])
        assert np.array_equal(kn[b, o], st["norm"][i].astype(np.float16))
        assert np.array_equal(sc[b, o], st["vscale"][i].astype(np.float16))
        assert np.array_equal(zr[b, o], st["vmin"][i].astype(np.float16))
    # slot 4 (never mapped) and the padding are untouched
    assert (cache[1, 0] == 0xAB).all()
    assert (cache[..., g["raw"]:] == 0xAB).all()


def _rand_cache(rng, nb, bs, H, d, kb, vb, n_tok, v_rotate=False):
    g = O.v1_geometry(d, kb, vb)
    cache = np.zeros((nb, bs, H, max(g["slot"], 128)), np.uint8)
    k = rng.standard_normal((n_tok, H, d)).astype(np.float32)
    v = rng.standard_normal((n_tok, H, d)).astype(np.float32)
    c = O.lloyd_max_codebook(d, kb)[1].astype(np.float32)
    slots = rng.permutation(nb * bs)[:n_tok]
    O.v1_store(k, v, slots, cache, O.v1_midpoints(c), kb, vb, v_rotate=v_rotate)
    return cache, c, k, v, slots


@pytest.mark.parametrize("v_rotate", [False, True])
def test_decode_equals_dense_attention_in_original_domain(v_rotate):
    # <q M, k^> = <q, k^ M^T>: attention over the un-rotated reconstructions
    rng = np.random.default_rng(11)
    nb, bs, H, d, kb, vb, Hq, B = 12, 16, 2, 64, 4, 2, 4, 2
    cache, c, _, _, _ = _rand_cache(rng, nb, bs, H, d, kb, vb, nb * bs, v_rotate)
    bt = rng.permutation(nb).reshape(B, nb // B).astype(np.int32)
    seq = np.array([37, 96], np.int32)
    q = rng.standard_normal((B, Hq, d)).astype(np.float32)
    got = O.v1_decode_attention(q, cache, bt, seq, c, kb, vb, 1 / math.sqrt(d), v_rotate=v_rotate)
    k_hat, v_hat = O.v1_dequant(cache, d, kb, vb, c)
    M = O.sylvester(d) / math.sqrt(d)
    kd = np.zeros((B, H, 96, d))
    vd = np.zeros((B, H, 96, d))
    for b in range(B):
        for p in range(seq[b]):
            blk, off = bt[b, p // bs], p % bs
            kd[b, :, p] = k_hat[blk, off] @ M.T
            vd[b, :, p] = (v_hat[blk, off] @ M.T) if v_rotate else v_hat[blk, off]
    want = O.dense_decode_attention(q, kd, vd, seq, 1 / math.sqrt(d))
    assert np.allclose(got, want, atol=1e-9)


def test_decode_norm_correction_makes_unit_directions():
    rng = np.random.default_rng(2)
    cache, c, _, _, _ = _rand_cache(rng, 4, 16, 1, 128, 3, 3, 64)
    k_hat, _ = O.v1_dequant(cache, 128, 3, 3, c)
    kc, kn, *_ = O.v1_unpack(cache, 128, 3, 3)
    assert np.allclose(np.linalg.norm(k_hat, axis=-1), kn.astype(np.float64), rtol=1e-12)
    k_raw, _ = O.v1_dequant(cache, 128, 3, 3, c, norm_correction=False)
    assert not np.allclose(np.linalg.norm(k_raw, axis=-1), kn.astype(np.float64), rtol=1e-3)


def test_decode_kv_start_masks_prefix():
    rng = np.random.default_rng(3)
    nb, bs, H, d = 8, 16, 1, 64
    cache, c, _, _, _ = _rand_cache(rng, nb, bs, H, d, 3, 3, nb * bs)
    bt = np.arange(nb, dtype=np.int32)[None]
    q = rng.standard_normal((1, 2, d)).astype(np.float32)
    full = O.v1_decode_attention(q, cache, bt, np.array([100]), c, 3, 3, 0.125, kv_start=np.array([40]))
    # the same attention with positions 40..99 relabelled to 0..59
    bt2 = bt.copy()
    cache2 = np.zeros_like(cache)
    for p in range(40, 100):
        cache2[(p - 40) // bs, (p - 40) % bs] = cache[p // bs, p % bs]
    part = O.v1_decode_attention(q, cache2, bt2, np.array([60]), c, 3, 3, 0.125)
    assert np.allclose(full, part, atol=1e-12)
    empty = O.v1_decode_attention(q, cache, bt, np.array([40]), c, 3, 3, 0.125, kv_start=np.array([40]))
    assert not empty.any()


@pytest.mark.parametrize("kb,vb,floor", [(4, 2, 0.8), (4, 4, 0.93), (8, 8, 0.999)])
def test_decode_quality(kb, vb, floor):
    # the compressed attention tracks exact attention on the raw K/V, and
    # more bits track it more closely
    rng = np.random.default_rng(4)
    nb, bs, H, d, Hq = 16, 16, 1, 128, 4
    cache, c, k, v, slots = _rand_cache(rng, nb, bs, H, d, kb, vb, nb * bs)
    inv = np.argsort(slots)
    bt = np.arange(nb, dtype=np.int32)[None]
    q = rng.standard_normal((1, Hq, d)).astype(np.float32) * 3
    got = O.v1_decode_attention(q, cache, bt, np.array([nb * bs]), c, kb, vb, 1 / math.sqrt(d))
    kk = k[inv].transpose(1, 0, 2)[None]
    vv = v[inv].transpose(1, 0, 2)[None]
    want = O.dense_decode_attention(q, kk, vv, [nb * bs], 1 / math.sqrt(d))
    cos = np.sum(got * want) / np.linalg.norm(got) / np.linalg.norm(want)
    assert cos > floor, cos


@pytest.mark.parametrize("v_rotate", [False, True])
def test_hybrid_equals_two_phase_lse_merge(v_rotate):
    """v1_hybrid_decode_attention (one softmax over the union) against the
    reference's own construction (v1_backend.py:1131-1277): phase 1 dense
    attention over the fp16 prefix with its log-sum-exp (sequence 0 only),
    phase 2 the quantised decode from kv_start = P with its log-sum-exp,
    merged by exp(lse - max) weights."""
    rng = np.random.default_rng(21)
    nb, bs, H, d, kb, vb, Hq, B = 12, 16, 2, 64, 4, 2, 4, 2
    cache, c, _, _, _ = _rand_cache(rng, nb, bs, H, d, kb, vb, nb * bs, v_rotate)
    bt = rng.permutation(nb).reshape(B, nb // B).astype(np.int32)
    seq = np.array([90, 70], np.int32)
    P = 33
    pk = rng.standard_normal((48, H, d)).astype(np.float16)
    pv = rng.standard_normal((48, H, d)).astype(np.float16)
    q = rng.standard_normal((B, Hq, d)).astype(np.float32)
    sc = 1 / math.sqrt(d)
    got = O.v1_hybrid_decode_attention(q, pk, pv, P, cache, bt, seq, c, kb, vb, sc, v_rotate=v_rotate)

    G = Hq // H
    M = O.sylvester(d) / math.sqrt(d)
    k_hat, _ = O.v1_dequant(cache, d, kb, vb, c)
    o2 = O.v1_decode_attention(q, cache, bt, seq, c, kb, vb, sc, kv_start=np.full(B, P), v_rotate=v_rotate)
    want = np.zeros_like(got)
    for b in range(B):
        pos = np.arange(P, seq[b])
        for h in range(Hq):
            s2 = k_hat[bt[b][pos // bs], pos % bs, h // G] @ (q[b, h].astype(np.float64) @ M) * sc
            l2 = s2.max() + np.log(np.exp(s2 - s2.max()).sum())
            if b == 0:
                s1 = pk[:P, h // G].astype(np.float64) @ q[b, h].astype(np.float64) * sc
                w1 = np.exp(s1 - s1.max())
                o1 = (w1 / w1.sum()) @ pv[:P, h // G].astype(np.float64)
                l1 = s1.max() + np.log(w1.sum())
            else:
                o1, l1 = np.zeros(d), -np.inf
            m = max(l1, l2)
            e1, e2 = np.exp(l1 - m), np.exp(l2 - m)
            want[b, h] = (o1 * e1 + o2[b, h] * e2) / (e1 + e2)
    assert np.allclose(got, want, atol=1e-10)
    # sequence 1 sees no prefix: exactly the kv_start decode
    assert np.allclose(got[1], o2[1], atol=1e-12)


def test_v_lloyd_max_store_fields_and_codes():
    """TURBOQUANT_V_LLOYD_MAX (triton_inkernel_store.py:159-200): codes by brute
    force (#{K midpoints m : m <= v / (||v|| + 1e-8)}), the norm in the scale
    field, a zero min field; and 2/3-bit V fall through to the uniform codes."""
    rng = np.random.default_rng(31)
    d, kb, H, N = 128, 4, 2, 24
    c = O.lloyd_max_codebook(d, kb)[1].astype(np.float32)
    mids = O.v1_midpoints(c)
    g = O.v1_geometry(d, kb, 4)
    k = rng.standard_normal((N, H, d)).astype(np.float32)
    v = (rng.standard_normal((N, H, d)) * 3).astype(np.float32)
    cache = np.zeros((4, 8, H, g["slot"]), np.uint8)
    st = O.v1_store(k, v, np.arange(N), cache, mids, kb, 4, v_rotate=True, v_lloyd_max=True)
    vv = st["value"]  # rotated, as stored
    for i in range(0, N, 5):
        for h in range(H):
            x = vv[i, h].astype(np.float64)
            nrm = np.float32(np.sqrt((x * x).sum() + 1e-16))
            u = (vv[i, h] / (nrm + np.float32(1e-8))).astype(np.float32)
            want = np.array([sum(1 for m in mids if m <= e) for e in u])
            assert np.array_equal(st["vcodes"][i, h], want)
    kc, kn, vc, sc, zr = O.v1_unpack(cache, d, kb, 4)
    blk, off = np.arange(N) // 8, np.arange(N) % 8
    assert np.array_equal(sc[blk, off], st["vscale"].astype(np.float16))
    assert not zr[blk, off].any()
    # 3-bit V ignores the flag (uniform codes, as the reference's VQB == 4 test)
    g3 = O.v1_geometry(d, kb, 3)
    a = np.zeros((4, 8, H, g3["slot"]), np.uint8)
    b = np.zeros_like(a)
    O.v1_store(k, v, np.arange(N), a, mids, kb, 3, v_rotate=True)
    O.v1_store(k, v, np.arange(N), b, mids, kb, 3, v_rotate=True, v_lloyd_max=True)
    assert np.array_equal(a, b)


def test_v_lloyd_max_dequant_norm_and_quality():
    """Dequantised Lloyd-Max V (triton_decode_offset.py:399-419): the norm
    correction makes ||V^|| equal the stored fp16 norm, and V^ taken back by
    M^T tracks the original V (4-bit Lloyd-Max on unit directions)."""
    rng = np.random.default_rng(32)
    d, kb, H, N = 128, 4, 2, 40
    c = O.lloyd_max_codebook(d, kb)[1].astype(np.float32)
    g = O.v1_geometry(d, kb, 4)
    k = rng.standard_normal((N, H, d)).astype(np.float32)
    v = rng.standard_normal((N, H, d)).astype(np.float32)
    cache = np.zeros((5, 8, H, g["slot"]), np.uint8)
    O.v1_store(k, v, np.arange(N), cache, O.v1_midpoints(c), kb, 4, v_rotate=True, v_lloyd_max=True)
    _, v_hat = O.v1_dequant(cache, d, kb, 4, c, v_lloyd_max=True)
    _, _, _, sc, _ = O.v1_unpack(cache, d, kb, 4)
    assert np.allclose(np.linalg.norm(v_hat, axis=-1), sc.astype(np.float64), rtol=1e-12)
    M = O.sylvester(d) / math.sqrt(d)
    rec = v_hat.reshape(-1, H, d)[:N] @ M.T
    cos = np.sum(rec * v, axis=-1) / (np.linalg.norm(rec, axis=-1) * np.linalg.norm(v, axis=-1))
    assert cos.min() > 0.98


def test_planar_rotation_matrix():
    """The planar strategy's M (x M): orthogonal with determinant 1, nonzero
    only on the 2x2 diagonal blocks, and x M turns each coordinate pair by
    +theta_p: e_{2p} M = (cos, sin) on (2p, 2p+1), e_{2p+1} M = (-sin, cos)
    (the row-vector form of the reference's block [[c, s], [-s, c]],
    rotation/planar.py:32-52); the angles are 2 pi U[0, 1) from the seeded
    CPU generator, so every rank builds the same matrix."""
    import math as _m
    import torch
    from fused_turboquant import v1
    d = 128
    M = v1.planar_rotation(d).double().numpy()
    assert np.abs(M @ M.T - np.eye(d)).max() < 1e-6
    assert abs(np.linalg.det(M) - 1.0) < 1e-5
    blockmask = np.kron(np.eye(d // 2), np.ones((2, 2))).astype(bool)
    assert not M[~blockmask].any()
    theta = torch.rand(d // 2, generator=torch.Generator().manual_seed(42)).double().numpy() * 2 * _m.pi
    e = np.eye(d)
    for p in (0, 1, 17, 63):
        r0, r1 = e[2 * p] @ M, e[2 * p + 1] @ M
        assert np.allclose(r0[2 * p:2 * p + 2], [np.cos(theta[p]), np.sin(theta[p])], atol=1e-6)
        assert np.allclose(r1[2 * p:2 * p + 2], [-np.sin(theta[p]), np.cos(theta[p])], atol=1e-6)
    assert np.array_equal(v1.planar_rotation(d).numpy(), v1.planar_rotation(d).numpy())
    # the oracle's matrix path with M = H / sqrt(d) reproduces its Hadamard path
    rng = np.random.default_rng(0)
    k = rng.standard_normal((5, 2, d)).astype(np.float32)
    H = O.sylvester(d) / _m.sqrt(d)
    y0, n0 = O.v1_k_rotate(k)
    y1, n1 = O.v1_k_rotate(k, H)
    assert np.abs(y0 - y1).max() < 1e-6 and np.array_equal(n0, n1)



def test_rotor_rotation_matrix():
    """The rotor strategy's M (x M) at d = 128: orthogonal with determinant 1,
    3x3 blocks on the diagonal for coordinates 0..125 and a 2x2 Givens block
    on 126..127; each 3x3 block is the rotor sandwich's matrix: its trace is
    1 + 2 cos(a) and it leaves fixed the axis dual to the rotor's bivector,
    (b3, -b2, b1) (the closed form of the reference's rotor.py:96-124 entries)."""
    import torch
    from fused_turboquant import v1
    d = 128
    M = v1.rotor_rotation(d).double().numpy()
    assert np.abs(M @ M.T - np.eye(d)).max() < 1e-5
    assert abs(np.linalg.det(M) - 1.0) < 1e-4
    mask = np.zeros((d, d), bool)
    for g in range(42):
        mask[3 * g:3 * g + 3, 3 * g:3 * g + 3] = True
    mask[126:128, 126:128] = True
    assert not M[~mask].any()
    gen = torch.Generator().manual_seed(42)
    b = torch.randn(43, 3, generator=gen, dtype=torch.float32)[:42].double().numpy()
    b /= np.linalg.norm(b, axis=1, keepdims=True)
    a = torch.rand(43, generator=gen, dtype=torch.float32).double().numpy()[:42] * 2 * np.pi
    for g in (0, 7, 41):
        blk = M[3 * g:3 * g + 3, 3 * g:3 * g + 3]
        assert abs(np.trace(blk) - (1 + 2 * np.cos(a[g]))) < 1e-5
        axis = np.array([b[g, 2], -b[g, 1], b[g, 0]])  # dual of p12 e12 + p13 e13 + p23 e23
        assert np.allclose(axis @ blk, axis, atol=1e-5)


# ---- pins of the oracle's dtype rounding, the uniform V rounding and the
# ---- seeded rotation matrices


def _round_cases():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32) * np.float32(3)
    bits = x.view(np.uint32).copy()
    # exact bf16 ties (low half 0x8000) with even and odd kept halves, and one ulp either side
    tie = (bits[:512] & np.uint32(0xFFFF0000)) | np.uint32(0x8000)
    extra = np.concatenate([tie, tie + np.uint32(1), tie - np.uint32(1),
                            tie ^ np.uint32(0x10000)]).view(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.4028235e38, -3.4028235e38,
                        1e-40, -1e-40, 65504.0, 65520.0, 65519.996, 6e-8, 2.9e-8, 1e-45],
                       np.float32)
    # f16 ties: values exactly halfway between two f16 numbers
    h = rng.standard_normal(512).astype(np.float16)
    nxt = np.nextafter(h, np.float16(np.inf))
    htie = ((h.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)
    return np.concatenate([x, extra, special, htie[np.isfinite(htie)]])


@pytest.mark.parametrize("dt,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_round_dtype_matches_torch_conversion(dt, tdt):
    """v1_round_dtype (the value dtype round trip of the V pre-rotation) equals
    torch's own float32 -> bf16 / f16 -> float32 conversion bit for bit, on
    exact ties, ±inf, NaN, overflow, subnormals and signed zero."""
    x = _round_cases()
    got = O.v1_round_dtype(x, dt)
    want = torch.from_numpy(x).to(tdt).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("vb", [1, 2, 3, 4])
@pytest.mark.parametrize("step", [1.0, 2.0, 0.25])
def test_quantize_v_rounds_half_up_at_exact_halves(vb, step):
    """Uniform V codes are trunc((v - min) / scale + 0.5)
    (triton_inkernel_store.py:210, 235): a value exactly halfway between codes
    k and k + 1 takes k + 1 for every k (round half to even would take the even
    one).  min = 0 and max = top * step make the scale exactly `step`."""
    top = (1 << vb) - 1
    halves = (np.arange(top) + 0.5) * step
    v = np.zeros((1, 64), np.float32)
    v[0, 0] = 0.0
    v[0, 1] = top * step
    v[0, 2:2 + top] = halves
    q, sc, mn, _ = O.v1_quantize_v(v, vb)
    assert sc[0] == np.float32(step) and mn[0] == 0.0
    assert q[0, 0] == 0 and q[0, 1] == top
    assert list(q[0, 2:2 + top]) == list(range(1, top + 1))


@pytest.mark.parametrize("kind", ["planar", "rotor", "iso_fast", "iso_full"])
def test_rotation_matrices_equal_the_reference(kind):
    """The seeded matrices of the block-diagonal strategies and their [B, D]
    coefficients equal the reference's own (tests/golden/rotations.npz,
    written from vllm_plugin/rotation/*.py build_matrix / compute_coeffs)."""
    import os
    from conftest import GOLDEN
    from fused_turboquant import v1
    z = np.load(os.path.join(GOLDEN, "rotations.npz"))
    keys = [k for k in z.files if k.startswith(kind + "_") and not k.endswith("_coeffs")
            and k[len(kind) + 1:].isdigit()]
    assert keys
    for k in keys:
        d = int(k[len(kind) + 1:])
        m = v1.rotation_matrix(kind, d)
        assert np.array_equal(m.numpy(), z[k]), k
        c = v1.block_coeffs(m, v1.BLOCK_SIZES[kind])
        assert np.array_equal(c.numpy(), z[k + "_coeffs"]), k


@pytest.mark.parametrize("kind", ["planar", "rotor", "iso_fast", "iso_full"])
def test_blockdiag_rotate_equals_matrix_product(kind):
    """v1_blockdiag_rotate (the block coefficients' fused multiply-add chain)
    equals x M of the dense matrix to within 2 float32 ulps of the result's
    scale, and exactly where a block holds a single nonzero per column."""
    from fused_turboquant import v1
    rng = np.random.default_rng(7)
    for d in (64, 128, 256):
        m = v1.rotation_matrix(kind, d)
        B = v1.BLOCK_SIZES[kind]
        cf = v1.block_coeffs(m, B).numpy()
        x = rng.standard_normal((40, d)).astype(np.float32)
        got = O.v1_blockdiag_rotate(x, cf, B)
        want = x.astype(np.float64) @ m.numpy().astype(np.float64)
        scale = np.abs(x).max(axis=-1, keepdims=True) * B
        assert np.all(np.abs(got - want) <= 2 * np.spacing(scale.astype(np.float32)))
    cf = np.zeros((3, 12), np.float32)  # the identity with 3x3 blocks: coefficient 1 at j = e mod 3
    for e in range(12):
        cf[e % 3, e] = 1.0
    x = rng.standard_normal((5, 12)).astype(np.float32)
    assert np.array_equal(O.v1_blockdiag_rotate(x, cf, 3), x)


def test_fp8_e4m3_matches_torch_in_range_and_saturates():
    """The fp8-key conversion (reference triton_inkernel_store.py:76-82) is
    IEEE-style round to nearest even onto e4m3fn: equal to torch's own
    float8_e4m3fn cast for every value below 464 (subnormals, exact midpoints,
    powers of two), +-448 above (the reference's saturating cast), and the
    decode table equals torch's for all 256 bytes."""
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.standard_normal(40000).astype(np.float32) * s for s in (1e-3, 3e-2, 1, 40, 300)])
    vals = O.e4m3_to_f32(np.arange(127))
    mids = ((vals[:-1].astype(np.float64) + vals[1:]) / 2).astype(np.float32)  # exact ties
    x = np.concatenate([x, mids, -mids, vals, np.float32([0.0, -0.0, 2.0 ** -10, 463.5, 2.0 ** -6])])
    got = O.f32_to_e4m3(x)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    inr = np.abs(x) < 464
    assert np.array_equal(got[inr], want[inr])
    big = np.float32([464.0, 1e4, np.inf, -np.inf, -500.0])
    assert np.array_equal(O.f32_to_e4m3(big), np.uint8([0x7E, 0x7E, 0x7E, 0xFE, 0xFE]))
    assert O.f32_to_e4m3(np.float32([np.nan]))[0] & 0x7F == 0x7F
    table = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    mine = O.e4m3_to_f32(np.arange(256))
    assert np.array_equal(np.isnan(mine), np.isnan(table))
    assert np.array_equal(mine[~np.isnan(mine)], table[~np.isnan(table)])


@pytest.mark.parametrize("d", [64, 128, 256])
def test_fp8_key_store_round_trip(d):
    """fp8 keys: the stored bytes decode to y * norm within half an fp8 step
    (3 mantissa bits: 2^-4 relative), no norm field, V region as for MSE keys."""
    rng = np.random.default_rng(d)
    k = rng.standard_normal((9, 2, d)).astype(np.float32) * 2
    v = rng.standard_normal((9, 2, d)).astype(np.float32)
    g = O.v1_geometry(d, 8, 8, key_fp8=True)
    assert g["kps"] == g["mse"] == d and g["raw"] == 2 * d + 4
    cache = np.zeros((2, 8, 2, g["slot"]), np.uint8)
    st = O.v1_store(k, v, np.arange(9), cache, np.zeros(1, np.float32), 8, 8, key_fp8=True)
    kc, kn, vc, sc, zr = O.v1_unpack(cache, d, 8, 8, key_fp8=True)
    assert kn is None
    x = (st["y"] * st["norm"][..., None]).astype(np.float64)
    back = O.e4m3_to_f32(kc.reshape(-1, 2, d)[:9]).astype(np.float64)
    assert np.all(np.abs(back - x) <= 2.0 ** -4 * np.abs(x) + 2.0 ** -10)
    # y * norm is the rotated key itself: H k / sqrt(d) up to the 1e-8 in the normalisation
    hk = k.astype(np.float64) @ O.sylvester(d) / math.sqrt(d)
    assert np.abs(x - hk).max() <= 1e-5 * np.abs(hk).max()


@pytest.mark.parametrize("kb,vb,fp8", [(1, 1, False), (1, 4, False), (4, 1, False), (3, 2, False),
                                       (8, 8, False), (8, 8, True)])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_slot_bytes_agree_everywhere(d, kb, vb, fp8):
    """C ABI (ftq_v1_slot_bytes_flags), Python (v1.slot_bytes) and the oracle
    give the same slot bytes for every supported width."""
    import ctypes
    from fused_turboquant import _lib
    from fused_turboquant import v1
    L = _lib.lib()
    L.ftq_v1_slot_bytes_flags.restype = ctypes.c_int64
    L.ftq_v1_slot_bytes_flags.argtypes = [ctypes.c_int] * 4
    want = O.v1_geometry(d, kb, vb, key_fp8=fp8)["raw"]
    assert v1.slot_bytes(d, kb, vb, key_fp8=fp8) == want
    assert L.ftq_v1_slot_bytes_flags(d, kb, vb, 4 if fp8 else 0) == want


@pytest.mark.parametrize("kb,vb,fp8", [(0, 2, False), (5, 4, False), (8, 4, False), (4, 8, False),
                                       (4, 4, True), (2, 2, True)])
def test_unsupported_widths_rejected(kb, vb, fp8):
    import ctypes
    from fused_turboquant import _lib
    from fused_turboquant import v1
    L = _lib.lib()
    L.ftq_v1_slot_bytes_flags.restype = ctypes.c_int64
    L.ftq_v1_slot_bytes_flags.argtypes = [ctypes.c_int] * 4
    assert L.ftq_v1_slot_bytes_flags(128, kb, vb, 4 if fp8 else 0) == -1
    with pytest.raises(ValueError):
        v1.slot_bytes(128, kb, vb, key_fp8=fp8)


@pytest.mark.parametrize("kind", ["rht", "planar", "rotor", "iso_full"])
@pytest.mark.parametrize("dtype,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16), ("f32", torch.float32)])
def test_v_rotation_is_the_dense_product_up_to_counted_ties(kind, dtype, tdt):
    """The oracle's V pre-rotation is the reference's expression
    ``einsum('nhd,de->nhe', value.float(), M).to(value.dtype)``
    (v1_backend.py:736-740) with M the layer's float32 matrix: the dense
    matrix it builds equals the reference's Sylvester builder
    (rotation/hadamard.py:28-34) and the block-diagonal matrices, and V bytes
    quantised from torch's own float32 einsum and from the Sylvester
    butterflies (another float32 order) equal the oracle's in every vector
    that ``v1_v_tie_vectors`` does not flag.  A dropped 1/sqrt(d), a
    transposed M or a missing cast to the value dtype fails here."""
    from fused_turboquant import v1
    rng = np.random.default_rng(90)
    d, n, vb = 128, 6000, 3
    if kind == "rht":
        h = torch.tensor([[1.0]])
        while h.shape[0] < d:
            h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
        m_ref = (h / math.sqrt(d)).numpy()
        M = O.v1_dense_rotation(d)
    else:
        m_ref = v1.rotation_matrix(kind, d).numpy()
        M = O.v1_dense_rotation(d, blockdiag=(v1.block_coeffs(torch.from_numpy(m_ref), v1.BLOCK_SIZES[kind]).numpy(),
                                              v1.BLOCK_SIZES[kind]))
    assert np.array_equal(M, m_ref)
    v = rng.standard_normal((n, 1, d)).astype(np.float32)
    v[: n // 50] *= 8
    vt = torch.from_numpy(v).to(tdt)
    v = vt.float().numpy()
    vr = O.v1_rotate_value(v, M)
    want = O.v1_quantize_v(O.v1_round_dtype(vr.astype(np.float32), dtype), vb)
    flagged = O.v1_v_tie_vectors(vr, dtype, vb)
    assert flagged.mean() < 0.05
    others = [torch.einsum("nhd,de->nhe", vt.float(), torch.from_numpy(M)).to(tdt).float().numpy()]
    if kind == "rht":
        others.append(O.v1_round_dtype((O.fwht_unscaled(v) * O.fwht_scale(d)).astype(np.float32), dtype))
    for got_v in others:
        got = O.v1_quantize_v(got_v, vb)
        diff = (np.any(got[0] != want[0], axis=-1) | (got[1].astype(np.float16) != want[1].astype(np.float16))
                | (got[2].astype(np.float16) != want[2].astype(np.float16)))
        assert not (diff & ~flagged).any()
    # the oracle's store writes the same V fields
    cache = np.zeros((n // 16 + 1, 16, 1, 128), np.uint8)
    mids = O.v1_midpoints(O.lloyd_max_codebook(d, 3)[1].astype(np.float32))
    st = O.v1_store(v, v, np.arange(n), cache, mids, 3, vb, v_rotate=True, value_dtype=dtype,
                    blockdiag=None if kind == "rht" else (v1.block_coeffs(torch.from_numpy(m_ref),
                                                                           v1.BLOCK_SIZES[kind]).numpy(),
                                                          v1.BLOCK_SIZES[kind]))
    assert np.array_equal(st["vcodes"], want[0]) and np.array_equal(st["vscale"], want[1])
    assert np.allclose(st["vrot"], vr, rtol=0, atol=0)


def test_v_tie_vectors_flag_a_planted_rounding_tie():
    """A rotated value placed exactly on a bf16 rounding boundary flags its
    vector when it is the maximum; the vector whose maximum is the bf16 value
    1.0 itself, with no element near a boundary or a code edge, is not."""
    d, vb = 8, 2
    base = np.array([0.1, 0.5, -1.0, 0.3, 0.7, -0.45, 0.15, 1.0], np.float64)
    tie = base.copy()
    tie[7] = 1.0 + 2.0 ** -8  # halfway between the bf16 values 1 and 1 + 2^-7
    assert O.v1_v_tie_vectors(tie[None], "bf16", vb)[0]
    assert not O.v1_v_tie_vectors(base[None], "bf16", vb)[0]
