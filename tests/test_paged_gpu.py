"""Paged library-format store + decode attention on gfx950 vs the CPU oracle.

Store: the codes read back from the pages equal the oracle's encode of the same
vectors except at codebook-boundary ties; norms fp16 within 1e-3 relative.
Attention: against float64 dense softmax attention over the oracle's decode of
the stored codes; max abs error <= 2e-2, mean <= 2e-3 (bf16 tolerance).
"""
import math

import numpy as np
import pytest

import bench
import torch

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu
TIE_ULPS = 4  # a code may differ only within 4 float32 ulps of a boundary (oracle.tie_ulps)


def _quants(cache):
    return cache.k_quant, cache.v_quant


def _fill(cache, lens, bt, hkv, d, g, dev, dtype=torch.bfloat16, outliers=False):
    page = cache.page_size
    ks, vs = [], []
    for b, L in enumerate(lens):
        k = torch.randn(L, hkv, d, generator=g)
        v = torch.randn(L, hkv, d, generator=g)
        if outliers:  # 2% of tokens at 8x the typical norm
            sel = torch.rand(L, generator=g) < 0.02
            k[sel] *= 8
            v[sel] *= 8
        k, v = k.to(dtype), v.to(dtype)
        if L:
            pos = torch.arange(L)
            slots = bt[b].long()[pos // page] * page + pos % page
            cache.store(k.to(dev), v.to(dev), slots.to(dev))
        ks.append(k)
        vs.append(v)
    return ks, vs


def _decoded(tq, x, bits, d):
    s = tq.rotation.signs.cpu().numpy()
    p, n16, u, _ = O.encode(x.float().numpy(), s, tq.quantizer.boundaries.cpu().numpy(), bits)
    return O.decode(p, n16, tq.quantizer.levels.cpu().numpy(), s, bits, d), p, n16, u


def _check_store(cache, k, v, slots, d, bk, bv, page, tag):
    """Codes and norms read back from the pages against the oracle's encode of
    the same K / V (ties within TIE_ULPS of a boundary allowed)."""
    n, hkv = k.shape[0], k.shape[1]
    kc, vc, kn, vn = O.paged_unpack(cache.kv_cache.cpu().numpy(), d, bk, bv)
    ties = 0
    for src, codes, norms, tq, bits in ((k, kc, kn, cache.k_quant, bk), (v, vc, vn, cache.v_quant, bv)):
        _, p, n16, u = _decoded(tq, src.reshape(-1, d), bits, d)
        want = O.unpack(p, bits, d).reshape(n, hkv, d)
        u = u.reshape(n, hkv, d)
        n16 = n16.reshape(n, hkv)
        sl = slots.numpy()
        ok = sl >= 0
        blk, off = sl[ok] // page, sl[ok] % page
        got = codes[blk, :, off]  # [m, hkv, d]
        diff = got != want[ok]
        if diff.any():
            dist = O.tie_ulps(u[ok][diff], tq.quantizer.boundaries.cpu().numpy()[1:-1], d)
            assert dist.max() <= TIE_ULPS
            ties += int(diff.sum())
        gn = norms[blk, :, off].astype(np.float32)
        wn = n16[ok].astype(np.float32)
        assert np.all(np.abs(gn - wn) <= 1e-3 * np.abs(wn) + 1e-7)
    print(f"[store {tag} bk={bk} bv={bv} page={page}] ties={ties}")


@pytest.mark.parametrize("bk,bv", [(3, 3), (4, 2), (2, 4), (4, 4), (2, 2)])
@pytest.mark.parametrize("page", [16, 32])
@pytest.mark.parametrize("d,dtype", [(128, torch.bfloat16), (128, torch.float16), (256, torch.bfloat16),
                                     (128, torch.float32)])
def test_store_layout_parity(cuda, bk, bv, page, d, dtype):
    """Scattered slots: every group takes the per-token store (inside the
    matrix-core kernel for 16-bit input, the VALU kernel for fp32)."""
    from fused_turboquant.paged import PagedTurboQuantCache
    hkv, nblk = 2, 6
    g = torch.Generator().manual_seed(bk * 10 + bv + page + d)
    cache = PagedTurboQuantCache(nblk, page, hkv, d, bk, bv, device=cuda)
    n = nblk * page - 5  # leave a few slots untouched
    slots = torch.randperm(nblk * page, generator=g)[:n]
    slots[3] = -1  # skipped slot
    k = torch.randn(n, hkv, d, generator=g).to(dtype)
    v = torch.randn(n, hkv, d, generator=g).to(dtype)
    cache.store(k.to(cuda), v.to(cuda), slots.to(cuda))
    _check_store(cache, k, v, slots, d, bk, bv, page, "scattered")


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("n", [1, 5, 16, 17])
def test_store_decode_steps(cuda, d, n):
    """Decode-step sized stores (one token per sequence, a few sequences): no
    group is a whole sub-block, several steps in a row into the same pages."""
    from fused_turboquant.paged import PagedTurboQuantCache
    hkv, page, nblk, bk, bv = 4, 16, 24, 3, 3
    g = torch.Generator().manual_seed(500 + n + d)
    cache = PagedTurboQuantCache(nblk, page, hkv, d, bk, bv, device=cuda)
    ks, vs, ss = [], [], []
    for step in range(3):  # sequence i writes position `step` of page i
        slots = torch.arange(n) * page + step
        k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
        v = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16)
        cache.store(k.to(cuda), v.to(cuda), slots.to(cuda))
        ks.append(k)
        vs.append(v)
        ss.append(slots)
    _check_store(cache, torch.cat(ks), torch.cat(vs), torch.cat(ss), d, bk, bv, page, "decode steps")


@pytest.mark.parametrize("bk,bv", [(3, 3), (4, 2), (2, 4), (4, 4), (2, 2), (3, 4), (4, 3), (2, 3)])
@pytest.mark.parametrize("page", [16, 48])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [128, 256])
def test_store_prefill_parity(cuda, bk, bv, page, dtype, d):
    """A prefill: tokens in slot order over pages taken in a seeded order, so
    every full group of 16 fills one sub-block whole (the matrix-core store).
    Mixed in, in the same call: a group with a skipped slot, a group shifted
    off the sub-block boundary, and a ragged tail (the per-token store)."""
    from fused_turboquant.paged import PagedTurboQuantCache
    hkv, nblk = 3, 7
    g = torch.Generator().manual_seed(100 + bk * 10 + bv + page + d)
    cache = PagedTurboQuantCache(nblk, page, hkv, d, bk, bv, device=cuda)
    pages = torch.randperm(nblk, generator=g)
    slots = (pages[:, None] * page + torch.arange(page)[None, :]).reshape(-1)
    slots[16 * 2 + 5] = -1  # group 2: one skipped slot
    grp = slots[16 * 4:16 * 5].clone()  # group 4: one slot past the sub-block's start
    slots[16 * 4:16 * 5] = torch.cat([grp[1:], grp[:1]])
    n = slots.numel() - 7  # ragged tail
    slots = slots[:n]
    k = torch.randn(n, hkv, d, generator=g)
    v = torch.randn(n, hkv, d, generator=g)
    k[::37] *= 8  # a few outlier tokens
    k, v = k.to(dtype), v.to(dtype)
    cache.store(k.to(cuda), v.to(cuda), slots.to(cuda))
    _check_store(cache, k, v, slots, d, bk, bv, page, "prefill")


@pytest.mark.parametrize("case", range(16))
def test_store_random_shapes(cuda, case):
    """Seeded random store configurations: head_dim 128 / 256, K and V widths
    2..4, pages of 16..64 tokens, bf16 / fp16 / fp32 input, 1..8 kv heads,
    2..12 pages.  The slots run in page order (whole sub-blocks: the
    matrix-core store) with a seeded scattered stretch, skipped slots and a
    ragged tail (the per-token store); outlier keys in half the cases.
    Codes and norms against the oracle as in the fixed cases."""
    from fused_turboquant.paged import PagedTurboQuantCache
    rng = np.random.default_rng(7000 + case)
    d = int(rng.choice([128, 256]))
    bk, bv = int(rng.integers(2, 5)), int(rng.integers(2, 5))
    page = int(rng.choice([16, 32, 48, 64]))
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    hkv, nblk = int(rng.integers(1, 9)), int(rng.integers(2, 13))
    g = torch.Generator().manual_seed(7000 + case)
    cache = PagedTurboQuantCache(nblk, page, hkv, d, bk, bv, device=cuda)
    pages = torch.randperm(nblk, generator=g)
    slots = (pages[:, None] * page + torch.arange(page)[None, :]).reshape(-1)
    total = slots.numel()
    a = int(rng.integers(0, total))
    b = min(total, a + int(rng.integers(2, 40)))
    slots[a:b] = slots[a:b][torch.from_numpy(rng.permutation(b - a))]
    slots[torch.from_numpy(rng.choice(total, size=3, replace=False))] = -1
    n = int(rng.integers(1, total + 1))
    slots = slots[:n].clone()
    k = torch.randn(n, hkv, d, generator=g)
    v = torch.randn(n, hkv, d, generator=g)
    if rng.random() < 0.5:
        k[::29] *= 8
    k, v = k.to(dtype), v.to(dtype)
    cache.store(k.to(cuda), v.to(cuda), slots.to(cuda))
    _check_store(cache, k, v, slots, d, bk, bv, page,
                 f"random case={case} d={d} hkv={hkv} nblk={nblk} n={n} {dtype}")


@pytest.mark.parametrize("bk,bv", [(3, 3), (4, 2), (2, 4), (4, 4)])
@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (16, 2)])
def test_decode_attention_parity(cuda, bk, bv, hq, hkv):
    from fused_turboquant.paged import PagedTurboQuantCache
    d, page = 128, 16
    lens = [1, 17, 33, 100, 515, 1000]
    B = len(lens)
    maxp = max((L + page - 1) // page for L in lens)
    g = torch.Generator().manual_seed(bk * 100 + bv * 10 + hq)
    nblk = B * maxp + 3
    cache = PagedTurboQuantCache(nblk, page, hkv, d, bk, bv, device=cuda)
    bt = torch.randperm(nblk, generator=g)[: B * maxp].view(B, maxp).to(torch.int32)
    ks, vs = _fill(cache, lens, bt, hkv, d, g, cuda)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    S = max(lens)
    Kd = np.zeros((B, hkv, S, d))
    Vd = np.zeros((B, hkv, S, d))
    for b, L in enumerate(lens):
        Kd[b, :, :L] = _decoded(cache.k_quant, ks[b].reshape(-1, d), bk, d)[0].reshape(L, hkv, d).transpose(1, 0, 2)
        Vd[b, :, :L] = _decoded(cache.v_quant, vs[b].reshape(-1, d), bv, d)[0].reshape(L, hkv, d).transpose(1, 0, 2)
    ref = O.dense_decode_attention(q.float().numpy(), Kd, Vd, lens, 1 / math.sqrt(d))
    sl = torch.tensor(lens, dtype=torch.int32, device=cuda)
    for splits in (1, 3, 8):
        out = cache.decode_attention(q.to(cuda), bt.to(cuda), sl, num_splits=splits).float().cpu().numpy()
        err = np.abs(out - ref)
        print(f"[attn bk={bk} bv={bv} hq={hq} hkv={hkv} splits={splits}] max={err.max():.2e} mean={err.mean():.2e}")
        assert err.max() <= 2e-2 and err.mean() <= 2e-3
    for splits in (1, 2):  # fp32 output: the single-launch form (splits 1, GQA <= 4) and the split form
        out32 = cache.decode_attention(q.to(cuda), bt.to(cuda), sl, num_splits=splits,
                                       out=torch.empty(B, hq, d, device=cuda)).cpu().numpy()
        assert np.abs(out32 - ref).max() <= 2e-2


@pytest.mark.parametrize("bk,bv", [(3, 3), (4, 2), (2, 4)])
@pytest.mark.parametrize("hq,hkv", [(16, 4), (32, 4), (32, 2)])
def test_decode_attention_outlier_keys(cuda, bk, bv, hq, hkv):
    """Keys and values 8x the typical norm on 2% of tokens: large, spread-out
    scores, where a relative error in the scores (the f16 level table, the
    f16 query) moves softmax weights and outputs visibly.  Against float64
    attention over the oracle's decode; the bound grows with |want| by one
    bf16 ulp, as rounding the exact answer to bf16 alone errs by half of that."""
    from fused_turboquant.paged import PagedTurboQuantCache
    d, page = 128, 16
    lens = [1, 17, 100, 515, 1000]
    B = len(lens)
    maxp = max((L + page - 1) // page for L in lens)
    g = torch.Generator().manual_seed(500 + bk * 100 + bv * 10 + hq + hkv)
    nblk = B * maxp + 3
    cache = PagedTurboQuantCache(nblk, page, hkv, d, bk, bv, device=cuda)
    bt = torch.randperm(nblk, generator=g)[: B * maxp].view(B, maxp).to(torch.int32)
    ks, vs = _fill(cache, lens, bt, hkv, d, g, cuda, outliers=True)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    S = max(lens)
    Kd = np.zeros((B, hkv, S, d))
    Vd = np.zeros((B, hkv, S, d))
    for b, L in enumerate(lens):
        Kd[b, :, :L] = _decoded(cache.k_quant, ks[b].reshape(-1, d), bk, d)[0].reshape(L, hkv, d).transpose(1, 0, 2)
        Vd[b, :, :L] = _decoded(cache.v_quant, vs[b].reshape(-1, d), bv, d)[0].reshape(L, hkv, d).transpose(1, 0, 2)
    ref = O.dense_decode_attention(q.float().numpy(), Kd, Vd, lens, 1 / math.sqrt(d))
    sl = torch.tensor(lens, dtype=torch.int32, device=cuda)
    bound = 2e-2 + 2.0 ** -8 * np.abs(ref)
    for splits in (1, 3):
        out = cache.decode_attention(q.to(cuda), bt.to(cuda), sl, num_splits=splits).float().cpu().numpy()
        err = np.abs(out - ref)
        print(f"[attn outliers bk={bk} bv={bv} hq={hq} hkv={hkv} splits={splits}] max={err.max():.2e} "
              f"mean={err.mean():.2e} (|ref| max {np.abs(ref).max():.1f}) worst/bound {(err / bound).max():.2f}")
        assert (err <= bound).all() and err.mean() <= 2e-3 * max(1.0, float(np.abs(ref).mean()))


def test_decode_attention_page32_and_zero_len(cuda):
    from fused_turboquant.paged import PagedTurboQuantCache
    d, page, hq, hkv = 128, 32, 8, 2
    lens = [0, 5, 64, 77]
    B = len(lens)
    maxp = 3
    g = torch.Generator().manual_seed(9)
    cache = PagedTurboQuantCache(B * maxp, page, hkv, d, 3, 3, device=cuda)
    bt = torch.randperm(B * maxp, generator=g).view(B, maxp).to(torch.int32)
    ks, vs = _fill(cache, lens, bt, hkv, d, g, cuda)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    Kd = np.zeros((B, hkv, 77, d))
    Vd = np.zeros((B, hkv, 77, d))
    for b, L in enumerate(lens):
        if L:
            Kd[b, :, :L] = _decoded(cache.k_quant, ks[b].reshape(-1, d), 3, d)[0].reshape(L, hkv, d).transpose(1, 0, 2)
            Vd[b, :, :L] = _decoded(cache.v_quant, vs[b].reshape(-1, d), 3, d)[0].reshape(L, hkv, d).transpose(1, 0, 2)
    ref = O.dense_decode_attention(q.float().numpy(), Kd, Vd, lens, 1 / math.sqrt(d))
    for splits in (1, 4):  # single-launch form and split form
        out = cache.decode_attention(q.to(cuda), bt.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda),
                                     num_splits=splits).float().cpu().numpy()
        assert np.all(out[0] == 0), splits  # empty context -> zeros
        assert np.abs(out - ref).max() <= 2e-2, splits


def test_config3_full_size(cuda):
    """Config 3 at full size; two sequences checked against the oracle, the rest
    through the agreement of the default (the single-launch form: B * Hkv = 256
    workgroups of 16 waves) with the split form (4 splits + merge launch)."""
    from fused_turboquant import paged as P
    cache, q, bt, sl = bench.make_config3(cuda)
    B, hq, d = q.shape
    assert P.default_splits(B, cache.num_kv_heads, int(sl[0]), hq, d) == 1
    out = P.paged_decode_attention(q, cache.kv_cache, bt, sl, cache.k_quant, cache.v_quant)
    out4 = P.paged_decode_attention(q, cache.kv_cache, bt, sl, cache.k_quant, cache.v_quant, num_splits=4)
    a, b4 = out.float().cpu().numpy(), out4.float().cpu().numpy()
    assert np.isfinite(a).all()
    assert np.abs(a - b4).max() <= 1e-2
    kq, vq = cache.k_quant, cache.v_quant
    ctx = int(sl[0])
    full = cache.kv_cache.cpu().numpy()
    for bsel in (0, B - 1):
        kc, vc, kn, vn = O.paged_unpack(full[bt[bsel].cpu().numpy()], d, 3, 3)
        hkv = kc.shape[1]
        blocks = np.arange(kc.shape[0])
        Kd = np.zeros((1, hkv, ctx, d))
        Vd = np.zeros((1, hkv, ctx, d))
        for h in range(hkv):
            kcodes = kc[blocks, h].reshape(-1, d)[:ctx]
            vcodes = vc[blocks, h].reshape(-1, d)[:ctx]
            knr = kn[blocks, h].reshape(-1)[:ctx]
            vnr = vn[blocks, h].reshape(-1)[:ctx]
            Kd[0, h] = O.decode(O.pack(kcodes, 3), knr, kq.quantizer.levels.cpu().numpy(), kq.rotation.signs.cpu().numpy(), 3, d)
            Vd[0, h] = O.decode(O.pack(vcodes, 3), vnr, vq.quantizer.levels.cpu().numpy(), vq.rotation.signs.cpu().numpy(), 3, d)
        ref = O.dense_decode_attention(q[bsel:bsel + 1].float().cpu().numpy(), Kd, Vd, [ctx], 1 / math.sqrt(d))
        err = np.abs(a[bsel] - ref[0])
        print(f"[config3 seq {bsel}] max={err.max():.2e} mean={err.mean():.2e}")
        assert err.max() <= 2e-2 and err.mean() <= 2e-3


# ---- fp32-operand VALU form (ftq_paged_decode_attention_valu) ----------------


def _dense_ref(cache, lens, bt, q, bk, bv, d):
    """float64 attention over the oracle's decode of the codes and norms the
    GPU store wrote (read back from the pages), so store ties do not enter."""
    full = cache.kv_cache.cpu().numpy()
    kq, vq = cache.k_quant, cache.v_quant
    B = len(lens)
    hkv = full.shape[1]
    S = max(lens)
    Kd = np.zeros((B, hkv, S, d))
    Vd = np.zeros((B, hkv, S, d))
    for b, L in enumerate(lens):
        if not L:
            continue
        kc, vc, kn, vn = O.paged_unpack(full[bt[b].numpy()], d, bk, bv)
        for h in range(hkv):
            Kd[b, h, :L] = O.decode(O.pack(kc[:, h].reshape(-1, d)[:L], bk), kn[:, h].reshape(-1)[:L],
                                    kq.quantizer.levels.cpu().numpy(), kq.rotation.signs.cpu().numpy(), bk, d)
            Vd[b, h, :L] = O.decode(O.pack(vc[:, h].reshape(-1, d)[:L], bv), vn[:, h].reshape(-1)[:L],
                                    vq.quantizer.levels.cpu().numpy(), vq.rotation.signs.cpu().numpy(), bv, d)
    return O.dense_decode_attention(q.float().numpy(), Kd, Vd, lens, 1 / math.sqrt(d))


@pytest.mark.parametrize("case", range(20))
def test_decode_attention_random_shapes(cuda, case):
    """Seeded random configurations of the paged decode: head_dim 128 / 256,
    K and V widths 2..4, GQA group 1..16, page sizes 16..64, ragged contexts
    with empty rows, the single-launch and split forms (1..24 splits), bf16 /
    fp16 / fp32 queries and outputs; against float64 attention over the
    oracle's decode of the stored pages."""
    from fused_turboquant.paged import PagedTurboQuantCache
    rng = np.random.default_rng(2000 + case)
    d = int(rng.choice([128, 256]))
    bk, bv = int(rng.integers(2, 5)), int(rng.integers(2, 5))
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = hkv * int(rng.choice([1, 2, 3, 4, 8, 16]))
    page = int(rng.choice([16, 32, 48, 64]))
    B = int(rng.integers(1, 6))
    lens = [int(x) for x in rng.integers(0, 600, B)]
    lens[int(rng.integers(0, B))] = max(lens[0], 1)  # at least one non-empty row
    splits = int(rng.choice([1, 2, 3, 8, 24]))
    qdt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    odt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    maxp = max(1, max((L + page - 1) // page for L in lens))
    g = torch.Generator().manual_seed(case)
    nblk = B * maxp + 2
    cache = PagedTurboQuantCache(nblk, page, hkv, d, bk, bv, device=cuda)
    bt = torch.randperm(nblk, generator=g)[: B * maxp].view(B, maxp).to(torch.int32)
    _fill(cache, lens, bt, hkv, d, g, cuda)
    q = torch.randn(B, hq, d, generator=g).to(qdt)
    ref = _dense_ref(cache, lens, bt, q, bk, bv, d)
    sl = torch.tensor(lens, dtype=torch.int32, device=cuda)
    out = cache.decode_attention(q.to(cuda), bt.to(cuda), sl, num_splits=splits,
                                 out=torch.empty(B, hq, d, dtype=odt, device=cuda)).float().cpu().numpy()
    for b, L in enumerate(lens):
        if L == 0:
            assert not out[b].any()
    err = np.abs(out - ref)
    tag = (f"[paged random case={case} d={d} K{bk}V{bv} hq={hq} hkv={hkv} page={page} B={B} S={splits} "
           f"{qdt}->{odt}]")
    print(f"{tag} max={err.max():.2e} mean={err.mean():.2e}")
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, tag


@pytest.mark.parametrize("bk,bv", [(3, 3), (4, 2), (2, 4), (4, 4), (2, 2)])
@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (12, 4)])
@pytest.mark.parametrize("outliers", [False, True])
def test_decode_attention_fp32_operands(cuda, bk, bv, hq, hkv, outliers):
    """The fp32 VALU form takes every product in fp32, like the reference, so
    with a float32 output it matches float64 attention over the oracle's
    decode of the stored codes to fp32 rounding -- also with keys and values
    8x the typical norm on 2% of tokens, where the f16-operand kernel needs
    the bf16-ulp allowance."""
    from fused_turboquant.paged import PagedTurboQuantCache
    d, page = 128, 16
    lens = [0, 1, 17, 33, 100, 515, 1000]
    B = len(lens)
    maxp = max((L + page - 1) // page for L in lens)
    g = torch.Generator().manual_seed(1300 + bk * 100 + bv * 10 + hq + outliers)
    nblk = B * maxp + 3
    cache = PagedTurboQuantCache(nblk, page, hkv, d, bk, bv, device=cuda)
    bt = torch.randperm(nblk, generator=g)[: B * maxp].view(B, maxp).to(torch.int32)
    _fill(cache, lens, bt, hkv, d, g, cuda, outliers=outliers)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    ref = _dense_ref(cache, lens, bt, q, bk, bv, d)
    sl = torch.tensor(lens, dtype=torch.int32, device=cuda)
    for splits in (1, 3, 8):
        out = cache.decode_attention(q.to(cuda), bt.to(cuda), sl, num_splits=splits, operands="fp32",
                                     out=torch.empty(B, hq, d, device=cuda)).cpu().numpy()
        err = np.abs(out - ref)
        print(f"[attn fp32 operands bk={bk} bv={bv} hq={hq} hkv={hkv} outliers={outliers} S={splits}] "
              f"max={err.max():.2e} mean={err.mean():.2e} (|ref| max {np.abs(ref).max():.1f})")
        assert np.all(out[0] == 0)
        assert (err <= 1e-4 + 1e-5 * np.abs(ref)).all()
        # bf16 output: only the output's rounding (at most 2^-8 of |x|) is added
        outb = cache.decode_attention(q.to(cuda), bt.to(cuda), sl, num_splits=splits,
                                      operands="fp32").float().cpu().numpy()
        errb = np.abs(outb - ref)
        assert (errb <= 1e-4 + 2.0 ** -8 * np.abs(ref)).all()


def test_fp32_operands_rejects_unsupported_shapes(cuda):
    from fused_turboquant.paged import PagedTurboQuantCache
    cache = PagedTurboQuantCache(4, 16, 2, 128, 3, 3, device=cuda)
    q = torch.zeros(1, 16, 128, dtype=torch.bfloat16, device=cuda)  # GQA 8
    bt = torch.zeros(1, 2, dtype=torch.int32, device=cuda)
    sl = torch.ones(1, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="at most 4 query heads"):
        cache.decode_attention(q, bt, sl, operands="fp32")
