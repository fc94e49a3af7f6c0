"""vLLM v1 slot formats beyond head_dim 128 with 2-4 bit codes, on gfx950 vs
the CPU oracle: 1-bit K or V (the k{K}v{V} aliases with a 1), 8-bit K and V
and fp8 keys (the 8-bit / fp8 boundary layers), head_dim 64 and 256, and the
fp32-operand decode kernel that serves them (and head_dim 128 on request).

Store: V codes, V scale / min (except counted V pre-rotation ties,
``oracle.v1_v_tie_vectors``), padding and unmapped slots byte-exact; K codes
exact except within 4 float32 ulps of a midpoint (code off by one); fp8 keys
exact except where y * norm lies within 4 float32 ulps of the midpoint
between two adjacent fp8 values; fp16 K norms within 1e-3.
Decode: against the oracle's float64 attention over cache bytes the oracle
wrote.  bf16 output: max <= 2e-2 + 2^-8 |want|, mean <= 2e-3 max(1, mean
|want|); fp32 output of the fp32 kernel: max <= 1e-4 max(1, |want|), the
products being the reference's own fp32 arithmetic.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from _v1_checks import check_v_region

pytestmark = pytest.mark.gpu
TIE_ULPS = 4
EXT_WIDTHS = [(1, 1), (1, 2), (1, 3), (1, 4), (2, 1), (3, 1), (4, 1), (8, 8)]


def _kv(g, n, h, d, dtype=torch.bfloat16, outliers=False):
    k = torch.randn(n, h, d, generator=g)
    v = torch.randn(n, h, d, generator=g)
    if outliers:
        sel = torch.rand(n, generator=g) < 0.02
        k[sel] *= 8
        v[sel] *= 8
    return k.to(dtype), v.to(dtype)


def _fp8_ties_ok(x, gb, wb):
    """fp8 bytes gb (GPU) and wb (oracle) of the fp32 values x (oracle): equal,
    or adjacent with x within TIE_ULPS float32 ulps of their midpoint."""
    diff = gb != wb
    if not diff.any():
        return 0, 0.0
    gv = O.e4m3_to_f32(gb[diff]).astype(np.float64)
    wv = O.e4m3_to_f32(wb[diff]).astype(np.float64)
    xs = x[diff].astype(np.float32)
    adj = np.abs(gb[diff].astype(int) - wb[diff].astype(int)) == 1
    mid = (gv + wv) / 2
    ulp = np.spacing(np.abs(xs)).astype(np.float64)
    dist = np.abs(xs.astype(np.float64) - mid) / ulp
    assert adj.all(), "fp8 bytes differ by more than one step"
    return int(diff.sum()), float(dist.max())


def _store_case(cuda, d, kb, vb, vrot, kind="rht", key_fp8=False, lloyd=False, seed=0):
    from fused_turboquant import v1
    nb, bs, h = 6, 16, 3
    g = torch.Generator().manual_seed(seed)
    layer = v1.TurboQuantV1Layer(d, kb, vb, v_rotate=vrot, kind=kind, key_fp8=key_fp8, v_lloyd_max=lloyd,
                                 device=cuda)
    cache = torch.full(layer.kv_cache_shape(nb, bs, h), 0xAB, dtype=torch.uint8, device=cuda)
    n = nb * bs - 5
    slots = torch.randperm(nb * bs, generator=g)[:n]
    slots[3] = -1
    k, v = _kv(g, n, h, d, outliers=True)
    layer.store(k.to(cuda), v.to(cuda), cache, slots.to(cuda))
    got = cache.cpu().numpy()
    want = np.full(got.shape, 0xAB, np.uint8)
    blockdiag = (layer.coeffs.cpu().numpy(), v1.BLOCK_SIZES[kind]) if layer.coeffs is not None else None
    mids = layer.midpoints.cpu().numpy()
    st = O.v1_store(k.float().numpy(), v.float().numpy(), slots.numpy(), want, mids, kb, vb, v_rotate=vrot,
                    value_dtype="bf16", v_lloyd_max=lloyd, blockdiag=blockdiag, key_fp8=key_fp8)
    geo = O.v1_geometry(d, kb, vb, key_fp8)
    sl = slots.numpy()
    ok = sl >= 0
    blk, off = sl[ok] // bs, sl[ok] % bs
    tag = f"d={d} kb={kb} vb={vb} vrot={vrot} {kind} fp8={key_fp8} lloyd={lloyd}"
    # V codes, V scale / min (up to V pre-rotation ties), padding and every unmapped slot
    check_v_region(got, want, st, ok, blk, off, geo, vrot or lloyd, "bf16", vb, lloyd=lloyd, tag=f"v1 ext store {tag}")
    unmapped = np.ones((nb, bs), bool)
    unmapped[blk, off] = False
    assert np.array_equal(got[unmapped], want[unmapped]), tag
    if key_fp8:
        x = (st["y"] * st["norm"][..., None]).astype(np.float32)[ok]
        ties, worst = _fp8_ties_ok(x, got[blk, off, :, :d], want[blk, off, :, :d])
        assert worst <= TIE_ULPS, (tag, worst)
        print(f"[v1 ext store {tag}] fp8 K ties={ties} max {worst:.2f} ulp")
        return
    gk = O.unpack(got[blk, off, :, :geo["mse"]], kb, d)
    wk = st["kcodes"][ok]
    diff = gk != wk
    worst = O.tie_ulps(st["y"][ok][diff], mids, d).max() if diff.any() else 0.0
    assert worst <= TIE_ULPS, (tag, worst)
    assert np.all(np.abs(gk[diff].astype(int) - wk[diff].astype(int)) == 1), tag
    gn = got[blk, off, :, geo["mse"]:geo["kps"]].copy().view(np.float16)[..., 0].astype(np.float32)
    wn = want[blk, off, :, geo["mse"]:geo["kps"]].copy().view(np.float16)[..., 0].astype(np.float32)
    assert np.all(np.abs(gn - wn) <= 1e-3 * np.abs(wn)), tag
    print(f"[v1 ext store {tag}] K ties={int(diff.sum())} of {wk.size}, max {worst:.2f} ulp")


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("kb,vb", EXT_WIDTHS)
def test_store_parity_ext_widths(cuda, d, kb, vb):
    _store_case(cuda, d, kb, vb, vrot=(kb + vb + d // 64) % 2 == 0, seed=d + 10 * kb + vb)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("vrot", [False, True])
def test_store_parity_fp8_keys(cuda, d, vrot):
    _store_case(cuda, d, 8, 8, vrot, key_fp8=True, seed=d + vrot)


@pytest.mark.parametrize("kind", ["planar", "rotor", "iso_full"])
@pytest.mark.parametrize("kb,vb,fp8", [(1, 3, False), (4, 1, False), (8, 8, False), (8, 8, True)])
def test_store_parity_ext_blockdiag(cuda, kind, kb, vb, fp8):
    _store_case(cuda, 128, kb, vb, vrot=True, kind=kind, key_fp8=fp8, seed=kb * 7 + vb)


@pytest.mark.parametrize("d", [64, 256])
def test_store_parity_lloyd_v_one_bit_keys(cuda, d):
    _store_case(cuda, d, 1, 4, vrot=True, lloyd=True, seed=d)


def _oracle_cache(g, nb, bs, h, d, kb, vb, vrot, key_fp8=False, lloyd=False, rotation=None, outliers=True):
    """Cache bytes written by the oracle (the decode tests do not depend on the
    GPU store); returns (cache, sorted centroids or None)."""
    from fused_turboquant import v1
    raw = v1.slot_bytes(d, kb, vb, key_fp8)
    cache = np.zeros((nb, bs, h, 1 << (raw - 1).bit_length()), np.uint8)
    k, v = _kv(g, nb * bs, h, d, outliers=outliers)
    c = None if key_fp8 else v1.default_centroids(d, kb).numpy()
    mids = np.zeros(1, np.float32) if key_fp8 else O.v1_midpoints(c)
    slots = torch.randperm(nb * bs, generator=g).numpy()
    O.v1_store(k.float().numpy(), v.float().numpy(), slots, cache, mids, kb, vb, v_rotate=vrot or lloyd,
               value_dtype="bf16", v_lloyd_max=lloyd, key_fp8=key_fp8, rotation=rotation)
    return cache, c


def _check(got, want, tag, fp32_out):
    err = np.abs(got.astype(np.float64) - want)
    if fp32_out:
        bound = 1e-4 * np.maximum(1.0, np.abs(want).max())
        print(f"[{tag}] fp32 out max {err.max():.2e} mean {err.mean():.2e} (bound {bound:.1e})")
        assert err.max() <= bound, tag
        return
    bound = 2e-2 + 2.0 ** -8 * np.abs(want)
    print(f"[{tag}] bf16 out max {err.max():.2e} mean {err.mean():.2e} worst/bound {(err / bound).max():.2f}")
    assert (err <= bound).all() and err.mean() <= 2e-3 * max(1.0, float(np.abs(want).mean())), tag


def _decode_case(cuda, d, kb, vb, hq, hkv, splits, vrot=True, key_fp8=False, lloyd=False, fp32_out=True,
                 operands="fp32", rotation=None, kv_start=False, seed=0):
    from fused_turboquant import v1
    nb, bs = 40, 16
    g = torch.Generator().manual_seed(seed)
    cache, c = _oracle_cache(g, nb, bs, hkv, d, kb, vb, vrot, key_fp8, lloyd,
                             None if rotation is None else rotation.numpy())
    lens = [0, 1, 17, 100, 257, 64, 400, 33]
    B = len(lens)
    mb = 26
    bt = torch.randint(0, nb, (B, mb), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g)
    sl = torch.tensor(lens, dtype=torch.int32)
    ks = torch.tensor([0, 0, 3, 50, 257, 0, 17, 32], dtype=torch.int32) if kv_start else None
    cent = torch.zeros(1) if c is None else torch.from_numpy(c)
    out = torch.empty(B, hq, d, device=cuda) if fp32_out else None
    res = v1.v1_decode_attention(q.to(torch.bfloat16).to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda),
                                 sl.to(cuda), cent.to(cuda), kb, vb, v_rotate=vrot, v_lloyd_max=lloyd,
                                 num_splits=splits, out=out, key_fp8=key_fp8, operands=operands,
                                 kv_start=None if ks is None else ks.to(cuda),
                                 rotation=None if rotation is None else rotation.to(cuda))
    want = O.v1_decode_attention(q.to(torch.bfloat16).float().numpy(), cache, bt.numpy(), sl.numpy(),
                                 c, kb, vb, 1 / math.sqrt(d), kv_start=None if ks is None else ks.numpy(),
                                 v_rotate=vrot or lloyd, v_lloyd_max=lloyd, key_fp8=key_fp8,
                                 rotation=None if rotation is None else rotation.numpy())
    got = res.float().cpu().numpy()
    assert not got[0].any()  # empty sequence -> zeros
    if kv_start:
        assert not got[4].any()  # kv_start == seq_len -> nothing attended
    _check(got, want, f"v1 decode d={d} kb={kb} vb={vb} hq={hq} hkv={hkv} S={splits} fp8={key_fp8} "
                      f"lloyd={lloyd} {operands}", fp32_out)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("kb,vb", EXT_WIDTHS + [(2, 2), (3, 3), (4, 2)])
def test_decode_parity_ext_widths(cuda, d, kb, vb):
    hq, hkv = [(8, 2), (4, 4), (16, 1)][(kb + vb) % 3]
    _decode_case(cuda, d, kb, vb, hq, hkv, splits=[1, 3, 8][(d // 64 + kb) % 3], vrot=(kb + d // 64) % 2 == 0,
                 seed=d * 10 + kb * 3 + vb)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (12, 2), (16, 1)])
def test_decode_parity_fp8_keys(cuda, d, hq, hkv):
    _decode_case(cuda, d, 8, 8, hq, hkv, splits=5, vrot=hq % 8 == 0, key_fp8=True, kv_start=True, seed=d + hq)


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("kb", [1, 2, 4])
def test_decode_parity_lloyd_v(cuda, d, kb):
    _decode_case(cuda, d, kb, 4, 8, 2, splits=4, lloyd=True, seed=d + kb)


@pytest.mark.parametrize("case", range(16))
def test_decode_random_formats(cuda, case):
    """Seeded random configurations of the fp32-product decode over every
    slot format: head_dim 64 / 128 / 256; K / V widths from 1..4 and 8, fp8
    keys, or Lloyd-Max V at 4 bits; GQA groups 1..16; 1..16 splits; V
    rotated or not; fp32 or bf16 output; with or without kv_start."""
    rng = np.random.default_rng(11000 + case)
    d = int(rng.choice([64, 128, 256]))
    fmt = int(rng.integers(0, 4))
    fp8 = lloyd = False
    if fmt == 0:
        kb, vb = EXT_WIDTHS[int(rng.integers(0, len(EXT_WIDTHS)))]
    elif fmt == 1:
        kb = vb = 8
        fp8 = True
    elif fmt == 2:
        kb, vb, lloyd = int(rng.integers(1, 5)), 4, True
    else:
        kb, vb = int(rng.integers(2, 5)), int(rng.integers(2, 5))
    hkv = int(rng.choice([1, 2, 4]))
    hq = hkv * int(rng.choice([1, 2, 3, 4, 8, 16]))
    splits = int(rng.choice([1, 2, 5, 16]))
    vrot = lloyd or bool(rng.random() < 0.5)
    _decode_case(cuda, d, kb, vb, hq, hkv, splits, vrot=vrot, key_fp8=fp8, lloyd=lloyd,
                 fp32_out=bool(rng.random() < 0.5), operands="fp32", kv_start=bool(rng.random() < 0.5),
                 seed=11000 + case)


@pytest.mark.parametrize("d", [64, 256])
def test_decode_bf16_out_and_kv_start(cuda, d):
    _decode_case(cuda, d, 3, 3, 8, 2, splits=16, fp32_out=False, kv_start=True, seed=d * 3)


@pytest.mark.parametrize("kind", ["planar", "rotor"])
def test_decode_parity_rotation_d256(cuda, kind):
    from fused_turboquant import v1
    m = v1.rotation_matrix(kind, 256)
    _decode_case(cuda, 256, 4, 2, 8, 2, splits=16, rotation=m, seed=11)


@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3), (2, 4)])
@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (16, 1)])
def test_fp32_operands_head_dim_128(cuda, kb, vb, hq, hkv):
    """operands="fp32" at head_dim 128: the reference's fp32 arithmetic, to
    fp32 rounding of the float64 oracle; the default matrix-core form agrees
    with it to its own (bf16-output) tolerance."""
    _decode_case(cuda, 128, kb, vb, hq, hkv, splits=6, seed=kb * 5 + vb + hq)
    _decode_case(cuda, 128, kb, vb, hq, hkv, splits=6, fp32_out=False, operands="f16", seed=kb * 5 + vb + hq)


def test_store_then_decode_boundary_modes(cuda):
    """GPU store then GPU decode, 8-bit MSE and fp8 keys, d=128 and 256,
    against the oracle's decode of the bytes the GPU wrote."""
    from fused_turboquant import v1
    for d in (128, 256):
        for fp8 in (False, True):
            g = torch.Generator().manual_seed(d + fp8)
            bs, hkv, hq = 16, 2, 8
            layer = v1.TurboQuantV1Layer(d, 8, 8, v_rotate=True, key_fp8=fp8, device=cuda)
            lens = [300, 45]
            nb = sum((L + bs - 1) // bs for L in lens) + 2
            cache = torch.zeros(layer.kv_cache_shape(nb, bs, hkv), dtype=torch.uint8, device=cuda)
            perm = torch.randperm(nb, generator=g).to(torch.int32)
            mb = max((L + bs - 1) // bs for L in lens)
            bt = torch.zeros(len(lens), mb, dtype=torch.int32)
            used = 0
            for b, L in enumerate(lens):
                npg = (L + bs - 1) // bs
                bt[b, :npg] = perm[used:used + npg]
                used += npg
                k, v = _kv(g, L, hkv, d, outliers=True)
                pos = torch.arange(L)
                layer.store(k.to(cuda), v.to(cuda), cache, (bt[b].long()[pos // bs] * bs + pos % bs).to(cuda))
            q = torch.randn(len(lens), hq, d, generator=g)
            sl = torch.tensor(lens, dtype=torch.int32)
            out = layer.decode(q.to(cuda), cache, bt.to(cuda), sl.to(cuda), out=torch.empty(len(lens), hq, d,
                                                                                            device=cuda))
            c = None if fp8 else layer.centroids.cpu().numpy()
            want = O.v1_decode_attention(q.numpy(), cache.cpu().numpy(), bt.numpy(), sl.numpy(), c, 8, 8,
                                         1 / math.sqrt(d), v_rotate=True, key_fp8=fp8)
            _check(out.cpu().numpy(), want, f"v1 boundary store+decode d={d} fp8={fp8}", True)
