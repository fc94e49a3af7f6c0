"""Raw fp16 boundary-layer slots on gfx950 vs the CPU oracle.

Store: every slot byte equals the oracle's (fp16 round to nearest even of the
bf16 / f16 / f32 input, [K | V] layout); negative slots and padding untouched.
Decode attention: against the oracle's float64 attention over the same cache
bytes.  K and V are exact fp16, the query enters the MFMA as f16 hi + lo and P
stays fp32, so the error is the output rounding plus fp32 accumulation:
f32 output  max |err| <= 1e-4 + 1e-4 |want|;
bf16 output max |err| <= 2^-8 |want| + 1e-3 (one bf16 rounding).
"""
import math

import numpy as np
import pytest

import bench
import torch

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _check(got, want, out_dtype, tag):
    err = np.abs(got.astype(np.float64) - want)
    if out_dtype == torch.float32:
        bound = 1e-4 + 1e-4 * np.abs(want)
    else:
        bound = 1e-3 + 2.0 ** -8 * np.abs(want)
    print(f"[{tag}] max {err.max():.2e} mean {err.mean():.2e} worst/bound {(err / bound).max():.2f}", flush=True)
    assert (err <= bound).all(), tag


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_store_parity(cuda, dtype, d):
    from fused_turboquant import raw
    g = torch.Generator().manual_seed(d)
    n, hkv, nb, bs = 77, 3, 9, 16
    k = (torch.randn(n, hkv, d, generator=g) * 4).to(DT[dtype])
    v = torch.randn(n, hkv, d, generator=g).to(DT[dtype])
    if dtype == "f32":
        k[0, 0, :3] = torch.tensor([70000.0, 3e-6, -6e-8])
    slots = torch.randperm(nb * bs, generator=g)[:n]
    slots[::7] = -1
    slot = 4 * d + 32
    cache = torch.full((nb, bs, hkv, slot), 0x5A, dtype=torch.uint8)
    want = cache.numpy().copy()
    O.raw_store(k.float().numpy(), v.float().numpy(), slots.numpy(), want)
    got = cache.to(cuda)
    raw.raw_store(k.to(cuda), v.to(cuda), got, slots.to(cuda))
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def _oracle_cache(g, nb, bs, hkv, d, n_tok, slot=None):
    slot = slot or 4 * d
    cache = np.zeros((nb, bs, hkv, slot), np.uint8)
    k = torch.randn(n_tok, hkv, d, generator=g).numpy()
    v = torch.randn(n_tok, hkv, d, generator=g).numpy()
    slots = torch.randperm(nb * bs, generator=g)[:n_tok].numpy()
    O.raw_store(k, v, slots, cache)
    return cache


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4), (8, 2), (14, 2), (16, 2)])
@pytest.mark.parametrize("splits", [1, 3, 16])
def test_decode_parity(cuda, hq, hkv, splits):
    from fused_turboquant import raw
    d, bs, nb = 128, 16, 48
    g = torch.Generator().manual_seed(hq * 100 + hkv * 10 + splits)
    cache = _oracle_cache(g, nb, bs, hkv, d, nb * bs)
    lens = [0, 1, 15, 17, 100, 257, 16, 64]
    B = len(lens)
    bt = torch.randint(0, nb, (B, 20), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    want = O.raw_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), 1 / math.sqrt(d))
    for odt in (torch.bfloat16, torch.float32):
        out = torch.empty(B, hq, d, dtype=odt, device=cuda)
        raw.raw_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                                 num_splits=splits, out=out)
        got = out.float().cpu().numpy()
        assert not got[0].any()  # empty sequence -> zeros
        _check(got, want, odt, f"raw hq={hq} hkv={hkv} S={splits} out={odt}")


@pytest.mark.parametrize("bs", [16, 32, 64])
def test_decode_kv_start_block_size_and_padded_slot(cuda, bs):
    from fused_turboquant import raw
    d, hkv, hq = 128, 2, 8
    nb = 1024 // bs
    g = torch.Generator().manual_seed(bs)
    cache = _oracle_cache(g, nb, bs, hkv, d, nb * bs, slot=4 * d + 64)  # slot wider than the data
    lens = [300, 31, 1000, 64]
    starts = [40, 31, 999, 0]
    bt = torch.stack([torch.randperm(nb, generator=g)[: 1024 // bs].to(torch.int32) for _ in lens])
    q = torch.randn(len(lens), hq, d, generator=g, dtype=torch.float32)
    sl = torch.tensor(lens, dtype=torch.int32)
    ks = torch.tensor(starts, dtype=torch.int32)
    out = raw.raw_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                                   kv_start=ks.to(cuda), num_splits=5,
                                   out=torch.empty(len(lens), hq, d, device=cuda))
    want = O.raw_decode_attention(q.numpy(), cache, bt.numpy(), sl.numpy(), 1 / math.sqrt(d), kv_start=ks.numpy())
    got = out.cpu().numpy()
    assert not got[1].any()  # kv_start == seq_len -> nothing attended
    _check(got, want, torch.float32, f"raw kv_start bs={bs}")


@pytest.mark.parametrize("case", range(16))
def test_decode_random_shapes(cuda, case):
    """Seeded random raw-slot decode configurations: head_dim 64 / 128 / 256,
    GQA groups up to 8 (16 at 64 / 256), 1..6 sequences with ragged, empty and
    offset ranges (kv_start), 1..40 splits, block sizes 16..64, slots wider
    than the data, bf16 / fp16 / fp32 queries and outputs, against the oracle."""
    from fused_turboquant import raw
    rng = np.random.default_rng(9000 + case)
    d = int(rng.choice([64, 128, 256]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([x for x in (1, 2, 3, 4, 7, 8, 16) if x <= (8 if d == 128 else 16)]))
    hq = hkv * G
    bs = int(rng.choice([16, 32, 64]))
    B = int(rng.integers(1, 7))
    lens = [int(x) for x in rng.integers(0, 700, B)]
    starts = [int(rng.integers(0, L + 1)) if rng.random() < 0.4 else 0 for L in lens]
    splits = int(rng.choice([1, 2, 3, 7, 16, 40]))
    qdt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    odt = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(0, 3))]
    pad = int(rng.choice([0, 32, 64]))
    mb = max(1, max((L + bs - 1) // bs for L in lens))
    nb = mb * B + 3
    g = torch.Generator().manual_seed(9000 + case)
    cache = _oracle_cache(g, nb, bs, hkv, d, nb * bs, slot=4 * d + pad)
    bt = torch.stack([torch.randperm(nb, generator=g)[:mb] for _ in range(B)]).to(torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(qdt)
    sl, ks = torch.tensor(lens, dtype=torch.int32), torch.tensor(starts, dtype=torch.int32)
    out = torch.empty(B, hq, d, dtype=odt, device=cuda)
    raw.raw_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                             kv_start=ks.to(cuda), num_splits=splits, out=out)
    want = O.raw_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), 1 / math.sqrt(d),
                                  kv_start=ks.numpy())
    got = out.float().cpu().numpy()
    for b in range(B):
        if lens[b] <= starts[b]:
            assert not got[b].any()
    _check(got, want, odt, f"raw random case={case} d={d} B={B} hq={hq} hkv={hkv} bs={bs} S={splits} "
                           f"pad={pad} {qdt}->{odt}")


def test_store_then_decode_end_to_end(cuda):
    """GPU store, then GPU decode, against the oracle pipeline on the same inputs
    (large-magnitude outliers, bf16 input)."""
    from fused_turboquant import raw
    d, bs, hkv, hq = 128, 16, 4, 16
    g = torch.Generator().manual_seed(77)
    lens = [513, 77, 1024]
    nb = sum((L + bs - 1) // bs for L in lens) + 3
    cache = torch.zeros(nb, bs, hkv, 4 * d, dtype=torch.uint8, device=cuda)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    mb = max((L + bs - 1) // bs for L in lens)
    bt = torch.zeros(len(lens), mb, dtype=torch.int32)
    used = 0
    for b, L in enumerate(lens):
        npg = (L + bs - 1) // bs
        bt[b, :npg] = perm[used:used + npg]
        used += npg
        k = torch.randn(L, hkv, d, generator=g)
        v = torch.randn(L, hkv, d, generator=g)
        sel = torch.rand(L, generator=g) < 0.02
        k[sel] *= 8
        v[sel] *= 8
        pos = torch.arange(L)
        slots = bt[b].long()[pos // bs] * bs + pos % bs
        raw.raw_store(k.to(torch.bfloat16).to(cuda), v.to(torch.bfloat16).to(cuda), cache, slots.to(cuda))
    q = torch.randn(len(lens), hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    out = raw.raw_decode_attention(q.to(cuda), cache, bt.to(cuda), sl.to(cuda))
    want = O.raw_decode_attention(q.float().numpy(), cache.cpu().numpy(), bt.numpy(), sl.numpy(), 1 / math.sqrt(d))
    _check(out.float().cpu().numpy(), want, torch.bfloat16, "raw store+decode")


def test_bench_shape_full_size(cuda):
    """The benchmark's shape (B=32, Hq=32, Hkv=8, ctx 8192, 512-byte slots,
    1.07 GB of K/V): oracle on two sequences, split-count invariance over all."""
    from fused_turboquant import raw
    setup = bench.raw_setup(cuda)
    setup["run"]()
    bench.check_lean(setup["run"])
    out = setup["out"].float().cpu().numpy()
    cache, bt, sl, q = setup["cache"], setup["bt"], setup["sl"], setup["q"]
    for b in (0, 31):
        sub = cache[bt[b].long()].cpu().numpy()  # the sequence's pages, in order
        want = O.raw_decode_attention(q[b:b + 1].float().cpu().numpy(), sub,
                                      np.arange(sub.shape[0], dtype=np.int32)[None], sl[b:b + 1].cpu().numpy(),
                                      1 / math.sqrt(128))
        _check(out[b:b + 1], want, torch.bfloat16, f"raw bench shape b={b}")
    other = raw.raw_decode_attention(q, cache, bt, sl, num_splits=1).float().cpu().numpy()
    _check(other, out.astype(np.float64), torch.bfloat16, "raw split invariance")


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (16, 1), (6, 3)])
def test_decode_parity_head_dims_64_256(cuda, d, hq, hkv):
    """Head dims 64 and 256 run the fp32 VALU kernel over the same raw slots
    (fp32 products: the reference's boundary_fp16_decode_attention arithmetic),
    with kv_start, empty rows and GQA groups up to 16; same bounds."""
    from fused_turboquant import raw
    bs, nb = 16, 48
    g = torch.Generator().manual_seed(d + hq)
    cache = _oracle_cache(g, nb, bs, hkv, d, nb * bs)
    lens = [0, 1, 15, 17, 100, 257, 16, 300]
    starts = [0, 0, 3, 17, 40, 0, 1, 256]
    B = len(lens)
    bt = torch.randint(0, nb, (B, 20), generator=g, dtype=torch.int32)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    ks = torch.tensor(starts, dtype=torch.int32)
    want = O.raw_decode_attention(q.float().numpy(), cache, bt.numpy(), sl.numpy(), 1 / math.sqrt(d),
                                  kv_start=ks.numpy())
    for odt, splits in ((torch.bfloat16, 3), (torch.float32, 16)):
        out = torch.empty(B, hq, d, dtype=odt, device=cuda)
        raw.raw_decode_attention(q.to(cuda), torch.from_numpy(cache).to(cuda), bt.to(cuda), sl.to(cuda),
                                 kv_start=ks.to(cuda), num_splits=splits, out=out)
        got = out.float().cpu().numpy()
        assert not got[0].any() and not got[3].any()  # empty row, kv_start == seq_len
        _check(got, want, odt, f"raw d={d} hq={hq} hkv={hkv} S={splits} out={odt}")
