"""Pins the oracle's raw fp16 slot functions (boundary layers, reference
vllm_plugin/v1_backend.py:1449-1545, triton_boundary_attn.py:28-219) without a GPU:
the store's fp16 rounding equals torch's .to(float16) (the reference's call),
including overflow, subnormals and exact halfway ties; the slot layout
[K fp16 | V fp16] round-trips; skipped slots stay untouched; the attention
equals a dense softmax computed from the K/V arrays themselves (so the block
table walk, the GQA head map and kv_start masking are checked independently)."""
import math

import numpy as np
import torch

from oracle import tq_oracle as O


def test_store_rounding_matches_torch_half():
    rng = np.random.default_rng(0)
    d, hkv, n = 128, 2, 40
    k = rng.standard_normal((n, hkv, d)).astype(np.float32) * np.float32(3.0)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    # special values: overflow, subnormal range, exact halfway points between fp16 neighbours
    k[0, 0, :4] = [70000.0, -1e6, 3e-6, -6e-8]
    h = np.float16(1.0)
    k[0, 0, 4] = np.float32(1.0) + np.float32(2.0 ** -11)       # halfway 1 and 1+2^-10 -> even (1.0)
    k[0, 0, 5] = np.float32(1.0) + np.float32(3 * 2.0 ** -11)   # halfway -> even (1+2^-9)
    cache = np.zeros((3, 16, hkv, 4 * d + 16), np.uint8)
    slots = np.arange(n, dtype=np.int64)
    O.raw_store(k, v, slots, cache)
    kt, vt = O.raw_unpack(cache, d)
    ref_k = torch.from_numpy(k).to(torch.float16).float().numpy()
    ref_v = torch.from_numpy(v).to(torch.float16).float().numpy()
    got_k = kt.reshape(-1, hkv, d)[:n]
    got_v = vt.reshape(-1, hkv, d)[:n]
    np.testing.assert_array_equal(got_k, ref_k)
    np.testing.assert_array_equal(got_v, ref_v)
    assert np.isinf(got_k[0, 0, 0]) and got_k[0, 0, 4] == 1.0 and got_k[0, 0, 5] == float(h + np.float16(2 ** -9))
    assert not cache[..., 4 * d:].any()  # padding untouched


def test_store_skips_negative_and_out_of_range_slots():
    rng = np.random.default_rng(1)
    d, hkv = 64, 1
    k = rng.standard_normal((4, hkv, d)).astype(np.float32)
    cache = np.full((2, 16, hkv, 4 * d), 0xAB, np.uint8)
    O.raw_store(k, k, np.array([-1, 5, 999, 31]), cache)
    kt, _ = O.raw_unpack(cache, d)
    assert np.array_equal(kt[0, 5, 0], k[1, 0].astype(np.float16).astype(np.float64))
    assert np.array_equal(kt[1, 15, 0], k[3, 0].astype(np.float16).astype(np.float64))
    untouched = np.ones((2, 16), bool)
    untouched[0, 5] = untouched[1, 15] = False
    assert (cache[untouched] == 0xAB).all()


def test_attention_equals_dense_softmax_over_the_arrays():
    rng = np.random.default_rng(2)
    d, hkv, G, bs, nb = 128, 2, 3, 16, 40
    lens, starts = [37, 0, 100, 16], [5, 0, 99, 0]
    B = len(lens)
    perm = rng.permutation(nb)
    bt = np.zeros((B, 8), np.int32)
    cache = np.zeros((nb, bs, hkv, 4 * d), np.uint8)
    K, V = [], []
    used = 0
    for b, L in enumerate(lens):
        npg = (L + bs - 1) // bs
        bt[b, :npg] = perm[used:used + npg]
        used += npg
        kb = rng.standard_normal((L, hkv, d)).astype(np.float16).astype(np.float32)
        vb = rng.standard_normal((L, hkv, d)).astype(np.float16).astype(np.float32)
        pos = np.arange(L)
        O.raw_store(kb, vb, bt[b][pos // bs].astype(np.int64) * bs + pos % bs, cache)
        K.append(kb.astype(np.float64))
        V.append(vb.astype(np.float64))
    q = rng.standard_normal((B, hkv * G, d))
    scale = 1 / math.sqrt(d)
    got = O.raw_decode_attention(q, cache, bt, np.array(lens), scale, kv_start=np.array(starts))
    for b, (L, s0) in enumerate(zip(lens, starts)):
        for h in range(hkv * G):
            if L <= s0:
                assert not got[b, h].any()
                continue
            sc = K[b][s0:L, h // G] @ q[b, h] * scale
            w = np.exp(sc - sc.max())
            want = (w / w.sum()) @ V[b][s0:L, h // G]
            np.testing.assert_allclose(got[b, h], want, rtol=1e-12, atol=1e-12)
