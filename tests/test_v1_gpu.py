"""vLLM v1 TURBOQUANT slot format on gfx950 vs the CPU oracle.

Store: every slot byte read back equals the oracle's store of the same vectors,
except K codes at midpoint ties (|y - midpoint| < 2e-6, code off by one; the
K norm is a float reduction whose order differs) and the fp16 K norm (within
1e-3 relative).  V codes, V scale and V min are bit-exact, except with V
rotated first (v_rotate): the reference rotates V by a dense float32 product
(v1_backend.py:736-740) whose summation order is its GEMM's, so a vector
whose rotated values sit within that order's spread of a rounding boundary
of the value dtype may differ; such vectors are counted and printed
(``oracle.v1_v_tie_vectors``).  Padding and unmapped slots stay untouched.
Decode attention: against the oracle's float64 attention over the same cache
bytes; max abs error <= 2e-2 + 2^-8 |want|, mean <= 2e-3 max(1, mean |want|)
(bf16 tolerance, widened by one bf16 ulp for large outputs).
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from _v1_checks import check_v_region

pytestmark = pytest.mark.gpu
TIE_ULPS = 4  # a code may differ only within 4 float32 ulps of a midpoint (oracle.tie_ulps)
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _kv(g, n, h, d, dtype, outliers=False):
    k = torch.randn(n, h, d, generator=g)
    v = torch.randn(n, h, d, generator=g)
    if outliers:
        sel = torch.rand(n, generator=g) < 0.02
        k[sel] *= 8
        v[sel] *= 8
    return k.to(dtype), v.to(dtype)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3), (2, 4), (4, 4), (2, 2)])
@pytest.mark.parametrize("vrot", [False, True])
def test_store_parity(cuda, d, kb, vb, vrot):
    dtn = "bf16" if (d + kb) % 2 == 0 else "f16"
    if d == 128 and kb == 3:
        dtn = "f32"
    _check_v1_store(cuda, d, kb, vb, vrot, dtn, 5, 16, 3, d * 100 + kb * 10 + vb + vrot)


@pytest.mark.parametrize("kb,vb", [(a, b) for a in (2, 3, 4) for b in (2, 3, 4)])
@pytest.mark.parametrize("dtn", ["bf16", "f16"])
@pytest.mark.parametrize("vrot", [False, True])
def test_store_parity_16bit_d128(cuda, kb, vb, dtn, vrot):
    """Every K, V width pair at d = 128 with bf16 and fp16 input, V rotated or
    not: 5 heads over 7 blocks of 16, skipped slots and outlier keys mixed in."""
    _check_v1_store(cuda, 128, kb, vb, vrot, dtn, 7, 16, 5, 900 + kb * 10 + vb + 2 * vrot, outliers=True)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3)])
@pytest.mark.parametrize("vrot", [False, True])
def test_store_zero_and_constant_vectors(cuda, d, kb, vb, vrot):
    """All-zero rows and rows the Hadamard transform maps to one nonzero
    element (constant +-1 rows, the alternating row): the rotated vectors hold
    exact zeros and their minimum or maximum is a zero. Every byte outside the
    K codes equals the oracle's (a rotated zero minimum is stored as +0, as
    the dense product gives it; an unrotated -0.0 minimum stays -0.0)."""
    _check_v1_store(cuda, d, kb, vb, vrot, "bf16", 3, 16, 2, 77 + d + kb + vrot, special=True)


@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3), (2, 4)])
@pytest.mark.parametrize("dtn", ["bf16", "f16"])
@pytest.mark.parametrize("vrot", [False, True])
def test_store_parity_matrix_core_path(cuda, kb, vb, dtn, vrot):
    """At least 32768 (token, head) vectors at d = 128 with 16-bit inputs take
    the matrix-core store: 4153 tokens x 8 heads (a partial last group of 16),
    skipped slots, outlier keys and the zero / constant rows, byte for byte
    against the oracle like the small cases."""
    _check_v1_store(cuda, 128, kb, vb, vrot, dtn, 260, 16, 8, 4400 + kb * 10 + vb + 2 * vrot, outliers=True,
                    special=True)


@pytest.mark.parametrize("case", range(16))
def test_store_random_shapes(cuda, case):
    """Seeded random store configurations: head_dim 64 / 128 / 256, K and V
    widths 2..4, V rotated or not, bf16 / fp16 / fp32 input, block sizes
    16..64, 1..12 heads, 2..40 blocks, outlier keys and the special rows;
    every slot byte against the oracle as in the fixed cases."""
    rng = np.random.default_rng(3000 + case)
    d = int(rng.choice([64, 128, 256]))
    kb, vb = int(rng.integers(2, 5)), int(rng.integers(2, 5))
    vrot = bool(rng.random() < 0.5)
    dtn = ["bf16", "f16", "f32"][int(rng.integers(0, 3))]
    bs = int(rng.choice([16, 32, 64]))
    h = int(rng.integers(1, 13))
    nb = int(rng.integers(2, 41))  # at least 17 slots: the checker skips slots 4 and 9
    _check_v1_store(cuda, d, kb, vb, vrot, dtn, nb, bs, h, 5000 + case, outliers=bool(rng.random() < 0.5),
                    special=bool(rng.random() < 0.3))


def _check_v1_store(cuda, d, kb, vb, vrot, dtn, nb, bs, h, seed, outliers=False, special=False):
    from fused_turboquant import v1
    g = torch.Generator().manual_seed(seed)
    layer = v1.TurboQuantV1Layer(d, kb, vb, v_rotate=vrot, device=cuda)
    slot = max(v1.slot_size(d, kb, vb), 128)
    cache = torch.full((nb, bs, h, slot), 0xAB, dtype=torch.uint8, device=cuda)
    n = nb * bs - 7
    slots = torch.randperm(nb * bs, generator=g)[:n]
    slots[4] = -1
    slots[9] = -5
    k, v = _kv(g, n, h, d, DT[dtn], outliers=outliers)
    if special:
        alt = torch.ones(d)
        alt[1::2] = -1
        # and a row whose minimum is -0.0 (every other element positive): without
        # the rotation that -0.0 is the stored minimum, fp16 0x8000
        negz = torch.rand(d, generator=g) + 0.25
        negz[3] = -0.0
        for i, row in zip((0, 1, 2, 3, 5, 6), (torch.zeros(d), torch.ones(d), -torch.ones(d), alt, -alt, negz)):
            k[i] = row.to(k.dtype)  # token 4 is the skipped one
            v[i] = row.to(v.dtype)
    layer.store(k.to(cuda), v.to(cuda), cache, slots.to(cuda))
    got = cache.cpu().numpy()

    want = np.full(got.shape, 0xAB, np.uint8)
    st = O.v1_store(k.float().numpy(), v.float().numpy(), slots.numpy(), want,
                    layer.midpoints.cpu().numpy(), kb, vb, v_rotate=vrot, value_dtype=dtn)
    geo = O.v1_geometry(d, kb, vb)
    # bytes outside the K region (K norm, V codes, V scale, V min, padding, unmapped slots)
    mse = geo["mse"]
    sl = slots.numpy()
    ok = sl >= 0
    blk, off = sl[ok] // bs, sl[ok] % bs
    check_v_region(got, want, st, ok, blk, off, geo, vrot, dtn, vb, tag=f"v1 store d={d} kb={kb} vb={vb} {dtn}")
    unmapped = np.ones((nb, bs), bool)
    unmapped[blk, off] = False
    assert np.array_equal(got[unmapped], want[unmapped])
    # K codes: equal except at midpoint ties
    gk = O.unpack(got[blk, off, :, :mse], kb, d)
    wk = st["kcodes"][ok]
    diff = gk != wk
    ties = int(diff.sum())
    if ties:
        y = st["y"][ok][diff]
        mids = layer.midpoints.cpu().numpy()
        worst = O.tie_ulps(y, mids, d).max()
        print(f"[v1 store d={d} kb={kb} vb={vb}] K ties={ties} max {worst:.2f} ulp")
        assert worst <= TIE_ULPS
        assert np.all(np.abs(gk[diff].astype(int) - wk[diff].astype(int)) == 1)
    # K norm fp16
    gn = got[blk, off, :, mse:mse + 2].copy().view(np.float16)[..., 0].astype(np.float32)
    wn = st["norm"][ok].astype(np.float16).astype(np.float32)
    assert np.all(np.abs(gn - wn) <= 1e-3 * np.abs(wn))
    print(f"[v1 store d={d} kb={kb} vb={vb} vrot={vrot} {dtn}] K code ties={ties} of {wk.size}")


def _oracle_cache(g, nb, bs, h, d, kb, vb, n_tok, vrot, dtype="bf16", outliers=False, lloyd=False):
    """Cache bytes written by the oracle (the decode tests do not depend on the GPU store)."""
    from fused_turboquant import v1
    slot = max(v1.slot_size(d, kb, vb), 128)
    cache = np.zeros((nb, bs, h, slot), np.uint8)
    k, v = _kv(g, n_tok, h, d, DT[dtype], outliers)
    c = v1.default_centroids(d, kb).numpy()
    slots = torch.randperm(nb * bs, generator=g)[:n_tok].numpy()
    O.v1_store(k.float().numpy(), v.float().numpy(), slots, cache, O.v1_midpoints(c), kb, vb,
               v_rotate=vrot or lloyd, value_dtype=dtype, v_lloyd_max=lloyd)
    return cache, c


def _check_attn(got, want, tag):
    """max |err| <= 2e-2 and mean |err| <= 2e-3 for outputs of magnitude <= 1;
    above that the bound grows with |want| by one bf16 ulp (2^-8 relative),
    since rounding the exact answer to bf16 alone errs by up to half of that
    (outlier tokens give outputs near 30, where a bf16 ulp is 0.125)."""
    err = np.abs(got.astype(np.float64) - want)
    bound = 2e-2 + 2.0 ** -8 * np.abs(want)
    mean_bound = 2e-3 * max(1.0, float(np.abs(want).mean()))
    print(f"[{tag}] max {err.max():.2e} mean {err.mean():.2e} (|want| max {np.abs(want).max():.2f}) "
          f"worst/bound {(err / bound).max():.2f}")
    assert (err <= bound).all() and err.mean() <= mean_bound, tag


@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3), (4, 4), (2, 2), (3, 4), (2, 3)])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 4), (16, 1), (16, 4), (32, 8)])
@pytest.mark.parametrize("splits", [1, 3, 16])
def test_decode_parity(cuda, kb, vb, hq, hkv, splits):
    from fused_turboquant import v1
    d, bs, nb = 128, 16, 48
    g = torch.Generator().manual_seed(kb * 1000 + vb * 100 + hq * 10 + splits)
    vrot = (kb + vb + splits) % 2 == 0
    cache, c = _oracle_cache(g, nb, bs, hkv, d, kb, vb, nb * bs, vrot)
    lens = [0, 1, 15, 17, 100, 257, 16, 64]
    B = len(lens)
    mb = 20
    bt = torch.randint(0, nb, (B, mb), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    out = v1.v1_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda),
                                 sl.to(cuda), torch.from_numpy(c).to(cuda), kb, vb,
                                 v_rotate=vrot, num_splits=splits)
    want = O.v1_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), c, kb, vb,
                                 1 / math.sqrt(d), v_rotate=vrot)
    assert out.dtype == torch.bfloat16
    got = out.float().cpu().numpy()
    assert not got[0].any()  # empty sequence -> zeros
    _check_attn(got, want, f"v1 attn kb={kb} vb={vb} hq={hq} hkv={hkv} S={splits} vrot={vrot}")


@pytest.mark.parametrize("hq,hkv", [(8, 2), (32, 8)])
@pytest.mark.parametrize("vrot,lloyd", [(False, False), (True, False), (True, True)])
@pytest.mark.parametrize("odt", ["f32", "bf16"])
def test_decode_single_split_direct_output(cuda, hq, hkv, vrot, lloyd, odt):
    """One split writes the output from the attention kernel (no merge launch):
    output and natural-log LSE against the merged two-split result (they
    differ only in the order of the partial sums) and the oracle, empty rows
    zero with LSE -inf, and the three-argument default split count
    (ftq_v1_default_splits) at 384+ (batch, kv head) units is that single
    split."""
    from fused_turboquant import v1
    d, bs, nb, kb = 128, 16, 48, 3
    vb = 4 if lloyd else 3
    g = torch.Generator().manual_seed(31 + hq + 2 * vrot + 4 * lloyd)
    cache, c = _oracle_cache(g, nb, bs, hkv, d, kb, vb, nb * bs, vrot, lloyd=lloyd)
    lens = [0, 1, 15, 17, 100, 257, 16, 64]
    starts = [0, 0, 3, 0, 99, 10, 16, 0]
    B = len(lens)
    bt = torch.randint(0, nb, (B, 20), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    sl, ks = torch.tensor(lens, dtype=torch.int32), torch.tensor(starts, dtype=torch.int32)
    res = {}
    for s in (1, 2):
        out = torch.full((B, hq, d), 7.0, dtype=DT[odt], device=cuda)
        lse = torch.full((B, hq), 7.0, device=cuda)
        v1.v1_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                               torch.from_numpy(c).to(cuda), kb, vb, v_rotate=vrot, v_lloyd_max=lloyd,
                               kv_start=ks.to(cuda), num_splits=s, out=out, lse=lse)
        res[s] = (out.float().cpu().numpy(), lse.cpu().numpy())
    (o1, l1), (o2, l2) = res[1], res[2]
    empty = [b for b in range(B) if lens[b] <= starts[b]]
    assert empty == [0, 6]
    for b in empty:
        assert not o1[b].any() and np.isneginf(l1[b]).all()
    live = [b for b in range(B) if b not in empty]
    assert np.isfinite(l1[live]).all()
    assert np.abs(l1[live] - l2[live]).max() <= 1e-5 * max(1.0, float(np.abs(l2[live]).max()))
    # the two splits start their running maxima, the f16 hi/lo parts of the
    # probabilities and the P.V offset terms at different tokens: fp32 sums in
    # another order (measured 7e-5 at |o| <= 3.2)
    tol = 5e-4 if odt == "f32" else 2.0 ** -7
    assert np.abs(o1 - o2).max() <= tol * max(1.0, float(np.abs(o2).max())), np.abs(o1 - o2).max()
    want = O.v1_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), c, kb, vb,
                                 1 / math.sqrt(d), kv_start=ks.numpy(), v_rotate=vrot, v_lloyd_max=lloyd)
    _check_attn(o1, want, f"v1 direct hq={hq} hkv={hkv} vrot={vrot} lloyd={lloyd} {odt}")
    assert v1.default_splits(48, 8, 4096) == 1 and v1.default_splits(4, 8, 131072) > 1


def test_choose_splits_fills_one_round(cuda):
    """The split factor with the slot format known (ftq_v1_choose_splits):
    the most splits whose workgroups the GPU holds at once -- 3 per CU for
    the GQA-4 kernel at K3 V3, 4 at K4 V2 -- with at least 8 tiles per wave.
    The values are the measured best split counts at these shapes (32 query /
    8 kv heads); the VALU formats keep the default rule."""
    from fused_turboquant import v1

    def ds(B, L, kb, vb, flags=v1.VROT):
        return v1.default_splits(B, 8, L, 32, 128, kb, vb, flags)
    assert ds(48, 2048, 3, 3) == 2 and ds(48, 32768, 3, 3) == 2
    assert ds(56, 8192, 3, 3) == 1 and ds(64, 2300, 3, 3) == 1
    assert ds(48, 2048, 4, 2) == 2 and ds(56, 8192, 4, 2) == 2 and ds(64, 8192, 4, 2) == 2
    assert ds(4, 131072, 4, 2) == 32
    assert ds(4, 1000, 4, 2) == 1  # 2 splits would leave under 8 tiles per wave
    assert ds(4, 131072, 4, 2, v1.VROT | v1.FP32) == v1.default_splits(4, 8, 131072)


@pytest.mark.parametrize("case", range(24))
def test_decode_random_shapes(cuda, case):
    """Seeded random configurations of the matrix-core decode: GQA group 1..16,
    K and V widths 2..4, V rotated or not (Lloyd-Max V at 4 bits), 1..40
    splits, block sizes 16..64, ragged contexts with empty and offset ranges
    (kv_start), bf16 / fp16 / fp32 queries and outputs, against the oracle."""
    from fused_turboquant import v1
    rng = np.random.default_rng(1000 + case)
    d = 128
    hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 3, 4, 8, 16]))
    hq = hkv * G
    kb, vb = int(rng.integers(2, 5)), int(rng.integers(2, 5))
    lloyd = vb == 4 and rng.random() < 0.5
    vrot = lloyd or rng.random() < 0.5
    bs = int(rng.choice([16, 32, 64]))
    B = int(rng.integers(1, 7))
    lens = [int(x) for x in rng.integers(0, 700, B)]
    starts = [int(rng.integers(0, L + 1)) if rng.random() < 0.4 else 0 for L in lens]
    splits = int(rng.choice([1, 2, 3, 7, 16, 40]))
    qdt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    odt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    mb = max(1, max((L + bs - 1) // bs for L in lens))
    nb = mb * B + 3
    g = torch.Generator().manual_seed(case)
    cache, c = _oracle_cache(g, nb, bs, hkv, d, kb, vb, nb * bs, vrot, lloyd=lloyd)
    bt = torch.stack([torch.randperm(nb, generator=g)[:mb] for _ in range(B)]).to(torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(qdt)
    sl, ks = torch.tensor(lens, dtype=torch.int32), torch.tensor(starts, dtype=torch.int32)
    out = torch.empty(B, hq, d, dtype=odt, device=cuda)
    v1.v1_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                           torch.from_numpy(c).to(cuda), kb, vb, v_rotate=vrot, v_lloyd_max=lloyd,
                           kv_start=ks.to(cuda), num_splits=splits, out=out)
    want = O.v1_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), c, kb, vb,
                                 1 / math.sqrt(d), kv_start=ks.numpy(), v_rotate=vrot, v_lloyd_max=lloyd)
    got = out.float().cpu().numpy()
    for b in range(B):
        if lens[b] <= starts[b]:
            assert not got[b].any()
    _check_attn(got, want, f"v1 random case={case} B={B} hq={hq} hkv={hkv} K{kb}V{vb} vrot={vrot} "
                           f"lloyd={lloyd} bs={bs} S={splits} {qdt}->{odt}")


@pytest.mark.parametrize("bs", [16, 32, 64])
def test_decode_kv_start_and_block_size(cuda, bs):
    from fused_turboquant import v1
    d, hkv, hq, kb, vb = 128, 2, 8, 4, 2
    nb = 1024 // bs
    g = torch.Generator().manual_seed(bs)
    cache, c = _oracle_cache(g, nb, bs, hkv, d, kb, vb, nb * bs, True)
    lens = [300, 31, 1000, 64]
    starts = [40, 31, 999, 0]
    bt = torch.stack([torch.randperm(nb, generator=g)[: 1024 // bs].to(torch.int32) for _ in lens])
    q = torch.randn(len(lens), hq, d, generator=g, dtype=torch.float32)
    sl = torch.tensor(lens, dtype=torch.int32)
    ks = torch.tensor(starts, dtype=torch.int32)
    out = v1.v1_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                                 torch.from_numpy(c).to(cuda), kb, vb, v_rotate=True, kv_start=ks.to(cuda),
                                 num_splits=5, out=torch.empty(len(lens), hq, d, device=cuda))
    want = O.v1_decode_attention(q.numpy(), cache, bt.numpy(), sl.numpy(), c, kb, vb, 1 / math.sqrt(d),
                                 kv_start=ks.numpy(), v_rotate=True)
    got = out.cpu().numpy()
    assert not got[1].any()  # kv_start == seq_len -> nothing attended
    _check_attn(got, want, f"v1 kv_start bs={bs}")


def test_store_then_decode_end_to_end(cuda):
    """GPU store followed by GPU decode against the oracle pipeline on the same inputs."""
    from fused_turboquant import v1
    d, bs, hkv, hq, kb, vb = 128, 16, 4, 16, 3, 3
    g = torch.Generator().manual_seed(77)
    layer = v1.TurboQuantV1Layer(d, kb, vb, v_rotate=True, device=cuda)
    lens = [513, 77, 1024]
    nb = sum((L + bs - 1) // bs for L in lens) + 3
    cache = torch.zeros(layer.kv_cache_shape(nb, bs, hkv), dtype=torch.uint8, device=cuda)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    mb = max((L + bs - 1) // bs for L in lens)
    bt = torch.zeros(len(lens), mb, dtype=torch.int32)
    used = 0
    for b, L in enumerate(lens):
        npg = (L + bs - 1) // bs
        bt[b, :npg] = perm[used:used + npg]
        used += npg
        k, v = _kv(g, L, hkv, d, torch.bfloat16, outliers=True)
        pos = torch.arange(L)
        slots = bt[b].long()[pos // bs] * bs + pos % bs
        layer.store(k.to(cuda), v.to(cuda), cache, slots.to(cuda))
    q = torch.randn(len(lens), hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    out = layer.decode(q.to(cuda), cache, bt.to(cuda), sl.to(cuda))
    want = O.v1_decode_attention(q.float().numpy(), cache.cpu().numpy(), bt.numpy(), sl.numpy(),
                                 layer.centroids.cpu().numpy(), kb, vb, 1 / math.sqrt(d), v_rotate=True)
    _check_attn(out.float().cpu().numpy(), want, "v1 store+decode")


def test_config4_full_size(cuda):
    """The v1 benchmark shape: K4V2, v_rotate, B=4, 32/8 heads, ctx ~ U[65536, 131072],
    2% of tokens x8.  Oracle on a subset of (sequence, kv head); split-count
    invariance over the whole output."""
    from fused_turboquant import v1
    d, bs, hkv, hq, kb, vb = 128, 16, 8, 32, 4, 2
    g = torch.Generator().manual_seed(4)
    lens = torch.randint(65536, 131073, (4,), generator=g).tolist()
    layer = v1.TurboQuantV1Layer(d, kb, vb, v_rotate=True, device=cuda)
    pages = [(L + bs - 1) // bs for L in lens]
    nb = sum(pages)
    cache = torch.zeros(layer.kv_cache_shape(nb, bs, hkv), dtype=torch.uint8, device=cuda)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.zeros(4, max(pages), dtype=torch.int32)
    used = 0
    gd = torch.Generator(device=cuda).manual_seed(5)
    for b, L in enumerate(lens):
        bt[b, :pages[b]] = perm[used:used + pages[b]]
        used += pages[b]
        btd = bt[b].to(cuda).long()
        for s0 in range(0, L, 32768):
            n = min(32768, L - s0)
            k = torch.randn(n, hkv, d, generator=gd, device=cuda)
            v = torch.randn(n, hkv, d, generator=gd, device=cuda)
            sel = torch.rand(n, generator=gd, device=cuda) < 0.02
            k[sel] *= 8
            v[sel] *= 8
            pos = torch.arange(s0, s0 + n, device=cuda)
            layer.store(k.to(torch.bfloat16), v.to(torch.bfloat16), cache, btd[pos // bs] * bs + pos % bs)
    q = torch.randn(4, hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    out = layer.decode(q.to(cuda), cache, bt.to(cuda), sl.to(cuda))
    f32 = [layer.decode(q.to(cuda), cache, bt.to(cuda), sl.to(cuda), num_splits=s,
                        out=torch.empty(4, hq, d, device=cuda)).cpu().numpy() for s in (8, 64)]
    o1 = out.float().cpu().numpy()
    assert np.isfinite(o1).all()
    # the split factor only changes the order of the final merge
    assert np.abs(f32[0] - f32[1]).max() <= 1e-3 * max(1.0, float(np.abs(f32[1]).max()))
    # oracle on (b, kv head) subsets: gather that head's slots into a small cache
    for b, kvh in ((0, 0), (3, 5)):
        L = lens[b]
        rows = bt[b, :pages[b]].long()
        sub = cache[rows.to(cuda)][:, :, kvh:kvh + 1].cpu().numpy()
        want = O.v1_decode_attention(q[b:b + 1, kvh * 4:kvh * 4 + 4].float().numpy(), sub,
                                     np.arange(pages[b], dtype=np.int32)[None], np.array([L]),
                                     layer.centroids.cpu().numpy(), kb, vb, 1 / math.sqrt(d),
                                     v_rotate=True)
        _check_attn(o1[b:b + 1, kvh * 4:kvh * 4 + 4], want, f"config4 b={b} kvh={kvh} ctx={L}")
        # the north-star bound itself (max <= 2e-2, mean <= 2e-3, no widening)
        # on the fp32 outputs, where no output rounding is added
        for s, o32 in zip((8, 64), f32):
            err = np.abs(o32[b:b + 1, kvh * 4:kvh * 4 + 4].astype(np.float64) - want)
            print(f"[config4 fp32 out S={s} b={b} kvh={kvh}] max {err.max():.2e} mean {err.mean():.2e}")
            assert err.max() <= 2e-2 and err.mean() <= 2e-3, (s, b, kvh)


@pytest.mark.parametrize("kb", [2, 3, 4])
def test_store_parity_v_lloyd_max(cuda, kb):
    """TURBOQUANT_V_LLOYD_MAX store (reference triton_inkernel_store.py:159-200):
    V rotated and rounded to bf16, Lloyd-Max codes of v / (||v|| + 1e-8) against
    the K midpoints, ||v|| in the scale field, 0 in the min field.  Codes equal
    the oracle's except at midpoint ties (the norms are float reductions whose
    order differs); both norms within 1e-3; every other byte exact."""
    from fused_turboquant import v1
    d, vb, nb, bs, h = 128, 4, 5, 16, 3
    g = torch.Generator().manual_seed(700 + kb)
    layer = v1.TurboQuantV1Layer(d, kb, vb, device=cuda, v_lloyd_max=True)
    assert layer.v_rotate
    slot = max(v1.slot_size(d, kb, vb), 128)
    cache = torch.full((nb, bs, h, slot), 0xAB, dtype=torch.uint8, device=cuda)
    n = nb * bs - 5
    slots = torch.randperm(nb * bs, generator=g)[:n]
    slots[3] = -1
    k, v = _kv(g, n, h, d, torch.bfloat16, outliers=True)
    layer.store(k.to(cuda), v.to(cuda), cache, slots.to(cuda))
    got = cache.cpu().numpy()
    want = np.full(got.shape, 0xAB, np.uint8)
    mids = layer.midpoints.cpu().numpy()
    st = O.v1_store(k.float().numpy(), v.float().numpy(), slots.numpy(), want, mids, kb, vb,
                    v_rotate=True, value_dtype="bf16", v_lloyd_max=True)
    geo = O.v1_geometry(d, kb, vb)
    sl = slots.numpy()
    ok = sl >= 0
    blk, off = sl[ok] // bs, sl[ok] % bs
    # padding, min field, unmapped slots: exact
    assert np.array_equal(got[..., geo["raw"]:], want[..., geo["raw"]:])
    assert np.array_equal(got[..., geo["kps"] + geo["vdb"] + 2:geo["raw"]],
                          want[..., geo["kps"] + geo["vdb"] + 2:geo["raw"]])
    unmapped = np.ones((nb, bs), bool)
    unmapped[blk, off] = False
    assert np.array_equal(got[unmapped], want[unmapped])
    gk, gkn, gv, gsc, gzr = O.v1_unpack(got, d, kb, vb)
    wk, wkn, wv, wsc, wzr = O.v1_unpack(want, d, kb, vb)
    assert not gzr[blk, off].any()
    # V vectors the float32 order of the pre-rotation can change (bf16
    # rounding ties of the rotated values) are counted and left out below
    vtie = O.v1_v_tie_vectors(st["vrot"][ok], "bf16", vb, v_lloyd_max=True)
    for name, gn, wn in (("K norm", gkn, wkn), ("V norm", gsc, wsc)):
        a, b = gn[blk, off].astype(np.float32), wn[blk, off].astype(np.float32)
        if name == "V norm":
            a, b = a[~vtie], b[~vtie]
        assert np.all(np.abs(a - b) <= 1e-3 * np.abs(b)), name
    vdiff = np.any(gv[blk, off] != wv[blk, off], axis=-1)
    print(f"[v1 store lloyd kb={kb}] V rotation ties: {int((vdiff & vtie).sum())} vectors differ, "
          f"{int(vtie.sum())} flagged of {vtie.size}")
    for name, gc, wc, u in (("K", gk, wk, st["y"]), ("V", gv, wv, st["vt"])):
        a, b = gc[blk, off], wc[blk, off]
        if name == "V":
            a, b, u = a[~vtie], b[~vtie], u[ok][~vtie]
        else:
            u = u[ok]
        diff = a != b
        if diff.any():
            assert O.tie_ulps(u[diff], mids, d).max() <= TIE_ULPS, name
            assert np.all(np.abs(a[diff].astype(int) - b[diff].astype(int)) == 1), name
        print(f"[v1 store lloyd kb={kb}] {name} code ties={int(diff.sum())} of {a.size}")


@pytest.mark.parametrize("kb,vb", [(2, 2), (2, 4), (3, 3), (4, 2)])
@pytest.mark.parametrize("hq,hkv", [(16, 4), (32, 4)])  # the GQA-4 kernel and the general one
@pytest.mark.parametrize("splits", [1, 5])
def test_decode_parity_outlier_keys(cuda, kb, vb, hq, hkv, splits):
    """Keys and values 8x the typical norm on 2% of tokens: large, spread-out
    scores, where a relative error in q.c / ||c|| of the centroid table's f16
    rounding (up to 2^-12, per centroid value) moves softmax weights by ~0.5%
    and the outputs by more than 2e-2.  Against the oracle's float64 attention."""
    from fused_turboquant import v1
    d, bs, nb = 128, 16, 48
    g = torch.Generator().manual_seed(700 + kb * 10 + vb + hq + splits)
    cache, c = _oracle_cache(g, nb, bs, hkv, d, kb, vb, nb * bs, (kb + vb) % 2 == 0, outliers=True)
    lens = [0, 1, 17, 100, 257, 64]
    starts = [0, 0, 5, 40, 0, 63]
    B = len(lens)
    bt = torch.randint(0, nb, (B, 20), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    ks = torch.tensor(starts, dtype=torch.int32)
    vrot = (kb + vb) % 2 == 0
    out = v1.v1_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                                 torch.from_numpy(c).to(cuda), kb, vb, v_rotate=vrot, kv_start=ks.to(cuda),
                                 num_splits=splits)
    want = O.v1_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), c, kb, vb,
                                 1 / math.sqrt(d), kv_start=ks.numpy(), v_rotate=vrot)
    got = out.float().cpu().numpy()
    assert not got[0].any()
    _check_attn(got, want, f"v1 outlier keys kb={kb} vb={vb} hq={hq} hkv={hkv} S={splits}")


@pytest.mark.parametrize("kb", [2, 3, 4])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (16, 4), (4, 4)])
@pytest.mark.parametrize("splits", [1, 5])
def test_decode_parity_v_lloyd_max(cuda, kb, hq, hkv, splits):
    """TURBOQUANT_V_LLOYD_MAX decode (reference triton_decode_offset.py:399-419):
    V = c[code] ||v||_16 / ||c[codes]||, un-rotated; against the oracle's float64
    attention over the same cache bytes, with kv_start on two rows."""
    from fused_turboquant import v1
    d, vb, bs, nb = 128, 4, 16, 48
    g = torch.Generator().manual_seed(900 + kb * 10 + hq + splits)
    cache, c = _oracle_cache(g, nb, bs, hkv, d, kb, vb, nb * bs, True, outliers=True, lloyd=True)
    lens = [0, 1, 17, 100, 257, 64]
    starts = [0, 0, 5, 40, 0, 63]
    B = len(lens)
    bt = torch.randint(0, nb, (B, 20), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    ks = torch.tensor(starts, dtype=torch.int32)
    out = v1.v1_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                                 torch.from_numpy(c).to(cuda), kb, vb, v_rotate=True, v_lloyd_max=True,
                                 kv_start=ks.to(cuda), num_splits=splits)
    want = O.v1_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), c, kb, vb,
                                 1 / math.sqrt(d), kv_start=ks.numpy(), v_rotate=True, v_lloyd_max=True)
    got = out.float().cpu().numpy()
    assert not got[0].any()
    _check_attn(got, want, f"v1 lloyd kb={kb} hq={hq} hkv={hkv} S={splits}")


@pytest.mark.parametrize("kind", ["planar", "rotor", "iso_fast", "iso_full"])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3), (2, 4)])
def test_store_parity_blockdiag(cuda, kind, d, kb, vb):
    """Block-diagonal store (planar / rotor / iso through their [B, d]
    coefficients; reference _fused_store_block_diag,
    triton_inkernel_store.py:649-860) against the oracle's restatement of the
    same fp32 arithmetic: K codes equal except within 4 ulps of a midpoint, K
    norms within 1e-3, V (rotated by the same blocks, rounded to bf16, min/max
    coded) byte for byte."""
    from fused_turboquant import v1
    bs, hkv, nb = 16, 4, 8
    n = nb * bs - 3
    g = torch.Generator().manual_seed(41 + kb + d)
    layer = v1.TurboQuantV1Layer(d, kb, vb, v_rotate=True, kind=kind, device=cuda)
    B = v1.BLOCK_SIZES[kind]
    cf = layer.coeffs.cpu().numpy()
    k, v = _kv(g, n, hkv, d, torch.bfloat16, outliers=True)
    slots = torch.randperm(nb * bs, generator=g)[:n]
    slots[5] = -1
    cache = torch.zeros(layer.kv_cache_shape(nb, bs, hkv), dtype=torch.uint8, device=cuda)
    layer.store(k.to(cuda), v.to(cuda), cache, slots.to(cuda))
    got = cache.cpu().numpy()
    want = np.zeros_like(got)
    mids = layer.midpoints.cpu().numpy()
    st = O.v1_store(k.float().numpy(), v.float().numpy(), slots.numpy(), want, mids, kb, vb,
                    v_rotate=True, value_dtype="bf16", blockdiag=(cf, B))
    geo = O.v1_geometry(d, kb, vb)
    sl = slots.numpy()
    ok = sl >= 0
    blk, off = sl[ok] // bs, sl[ok] % bs
    check_v_region(got, want, st, ok, blk, off, geo, True, "bf16", vb, tag=f"v1 {kind} store d={d} kb={kb} vb={vb}")
    gk = O.unpack(got[blk, off, :, :geo["mse"]], kb, d)
    wk = st["kcodes"][ok]
    diff = gk != wk
    worst = O.tie_ulps(st["y"][ok][diff], mids, d).max() if diff.any() else 0.0
    print(f"[v1 {kind} store d={d} kb={kb} vb={vb}] K ties={int(diff.sum())} max {worst:.2f} ulp")
    assert worst <= TIE_ULPS
    assert np.all(np.abs(gk[diff].astype(int) - wk[diff].astype(int)) == 1)
    gn = got[blk, off, :, geo["mse"]:geo["kps"]].copy().view(np.float16)[..., 0].astype(np.float32)
    wn = want[blk, off, :, geo["mse"]:geo["kps"]].copy().view(np.float16)[..., 0].astype(np.float32)
    assert np.all(np.abs(gn - wn) <= 1e-3 * np.abs(wn))


@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3)])
def test_store_parity_dense_matrix(cuda, kb, vb):
    """A caller's own d x d rotation (a seeded random orthogonal matrix) through
    the dense in-kernel product (ftq_v1_store_rot) against the oracle's x M in
    float64: K codes equal except where the rotated unit vector sits within
    1e-5 of a midpoint (the kernel's fp32 sum of d products is rounded
    differently), K norms within 1e-3, V within one code step."""
    from fused_turboquant import v1
    d, bs, hkv, nb = 128, 16, 4, 8
    n = nb * bs
    g = torch.Generator().manual_seed(45 + kb)
    M = torch.linalg.qr(torch.randn(d, d, generator=g, dtype=torch.float64))[0].to(torch.float32)
    layer = v1.TurboQuantV1Layer(d, kb, vb, v_rotate=True, rotation=M, device=cuda)
    k, v = _kv(g, n, hkv, d, torch.bfloat16)
    slots = torch.randperm(nb * bs, generator=g)[:n]
    cache = torch.zeros(layer.kv_cache_shape(nb, bs, hkv), dtype=torch.uint8, device=cuda)
    layer.store(k.to(cuda), v.to(cuda), cache, slots.to(cuda))
    got = cache.cpu().numpy()
    want = np.zeros_like(got)
    mids = layer.midpoints.cpu().numpy()
    O.v1_store(k.float().numpy(), v.float().numpy(), slots.numpy(), want, mids, kb, vb,
               v_rotate=True, value_dtype="bf16", rotation=M.numpy())
    kg, kng, vg, scg, zg = O.v1_unpack(got, d, kb, vb)
    kw, knw, vw, scw, zw = O.v1_unpack(want, d, kb, vb)
    y, _ = O.v1_k_rotate(k.float().numpy(), M.numpy())
    blk, off = slots.numpy() // bs, slots.numpy() % bs
    dk = kg[blk, off].astype(int) - kw[blk, off].astype(int)
    near = np.min(np.abs(y[..., None] - mids[None, None, None, :]), axis=-1) < 1e-5
    bad = (dk != 0) & ~((np.abs(dk) == 1) & near)
    print(f"[v1 dense store kb={kb} vb={vb}] K code ties={(dk != 0).sum()} of {dk.size}")
    assert not bad.any()
    kn_g, kn_w = kng[blk, off].astype(np.float64), knw[blk, off].astype(np.float64)
    assert np.abs(kn_g - kn_w).max() <= 1e-3 * np.abs(kn_w).max()
    vhg = vg[blk, off] * scg[blk, off][..., None].astype(np.float64) + zg[blk, off][..., None].astype(np.float64)
    vhw = vw[blk, off] * scw[blk, off][..., None].astype(np.float64) + zw[blk, off][..., None].astype(np.float64)
    step = np.maximum(scg[blk, off], scw[blk, off]).astype(np.float64)[..., None]
    assert (np.abs(vhg - vhw) <= 1.01 * step + 1e-3).all()


@pytest.mark.parametrize("kind", ["planar", "rotor", "iso_fast", "iso_full"])
@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 3), (2, 4)])
@pytest.mark.parametrize("hq,hkv", [(16, 4), (8, 1)])
def test_decode_parity_planar_matrix(cuda, kb, vb, hq, hkv, kind):
    """Matrix-strategy decode: q M in the kernel prologue and o M^T in the merge
    (reference rotation/matrix.py:47-48, v1_backend.py:1086-1092) against the
    oracle's float64 attention over the same cache bytes (written by the
    oracle with the same M)."""
    from fused_turboquant import v1
    d, bs, nb = 128, 16, 48
    g = torch.Generator().manual_seed(300 + kb * 10 + vb + hq)
    M = v1.rotation_matrix(kind, d).numpy()
    slot = max(v1.slot_size(d, kb, vb), 128)
    cache = np.zeros((nb, bs, hkv, slot), np.uint8)
    k, v = _kv(g, nb * bs, hkv, d, torch.bfloat16, outliers=True)
    c = v1.default_centroids(d, kb).numpy()
    slots = torch.randperm(nb * bs, generator=g).numpy()
    O.v1_store(k.float().numpy(), v.float().numpy(), slots, cache, O.v1_midpoints(c), kb, vb,
               v_rotate=True, value_dtype="bf16", rotation=M)
    lens = [0, 1, 17, 100, 257, 64]
    starts = [0, 0, 5, 40, 0, 63]
    B = len(lens)
    bt = torch.randint(0, nb, (B, 20), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    ks = torch.tensor(starts, dtype=torch.int32)
    for splits in (1, 5, 16):  # 16: the 4-wave-per-row merge with the o M^T un-rotation
        out = v1.v1_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                                     torch.from_numpy(c).to(cuda), kb, vb, v_rotate=True, kv_start=ks.to(cuda),
                                     num_splits=splits, rotation=torch.from_numpy(M).to(cuda))
        want = O.v1_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), c, kb, vb,
                                     1 / math.sqrt(d), kv_start=ks.numpy(), v_rotate=True, rotation=M)
        got = out.float().cpu().numpy()
        assert not got[0].any()
        _check_attn(got, want, f"v1 {kind} kb={kb} vb={vb} hq={hq} hkv={hkv} S={splits}")


@pytest.mark.parametrize("kind", ["planar", "rotor", "iso_full"])
@pytest.mark.parametrize("hq,hkv", [(16, 4), (8, 1)])
def test_decode_parity_v_lloyd_max_matrix(cuda, kind, hq, hkv):
    """Lloyd-Max V with a matrix strategy: the general kernel's VLM form with
    q M in its prologue and o M^T in the merge, against the oracle's float64
    attention over the same cache bytes (written by the oracle with the same
    M), 1, 5 and 16 splits."""
    from fused_turboquant import v1
    d, kb, vb, bs, nb = 128, 4, 4, 16, 48
    g = torch.Generator().manual_seed(950 + hq + hkv)
    M = v1.rotation_matrix(kind, d).numpy()
    slot = max(v1.slot_size(d, kb, vb), 128)
    cache = np.zeros((nb, bs, hkv, slot), np.uint8)
    k, v = _kv(g, nb * bs, hkv, d, torch.bfloat16, outliers=True)
    c = v1.default_centroids(d, kb).numpy()
    slots = torch.randperm(nb * bs, generator=g).numpy()
    O.v1_store(k.float().numpy(), v.float().numpy(), slots, cache, O.v1_midpoints(c), kb, vb,
               v_rotate=True, value_dtype="bf16", v_lloyd_max=True, rotation=M)
    lens = [0, 1, 17, 100, 257, 700]
    starts = [0, 0, 5, 40, 0, 63]
    B = len(lens)
    bt = torch.randint(0, nb, (B, 48), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    ks = torch.tensor(starts, dtype=torch.int32)
    want = O.v1_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), c, kb, vb,
                                 1 / math.sqrt(d), kv_start=ks.numpy(), v_rotate=True, v_lloyd_max=True,
                                 rotation=M)
    for splits in (1, 5, 16):
        out = v1.v1_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                                     torch.from_numpy(c).to(cuda), kb, vb, v_rotate=True, v_lloyd_max=True,
                                     kv_start=ks.to(cuda), num_splits=splits,
                                     rotation=torch.from_numpy(M).to(cuda))
        got = out.float().cpu().numpy()
        assert not got[0].any()
        _check_attn(got, want, f"v1 lloyd {kind} hq={hq} hkv={hkv} S={splits}")
