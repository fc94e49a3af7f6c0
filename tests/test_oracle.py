"""The CPU oracle pinned against the reference's own outputs and against
closed forms (reference tests/test_hadamard.py, tests/test_quantizer.py)."""
import math

import numpy as np
import pytest

from oracle import tq_oracle as O


def bf16_to_f32(u16):
    return (np.asarray(u16).astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("d", [2, 8, 64, 128, 256])
def test_fwht_matches_reference_outputs(golden, d):
    fw = golden["fwht"]
    assert np.array_equal(O.fwht(fw[f"x_{d}"]), fw[f"y_{d}"])


def test_fwht_known_answer_d2():
    # reference tests/test_hadamard.py:35-40
    y = O.fwht(np.array([[1.0, 0.0]], np.float32))
    assert np.allclose(y, [[1 / math.sqrt(2), 1 / math.sqrt(2)]], atol=1e-6)


@pytest.mark.parametrize("d", [4, 16, 64, 128])
def test_fwht_equals_sylvester_matrix(d):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((5, d)).astype(np.float32)
    ref = x.astype(np.float64) @ O.sylvester(d).T / math.sqrt(d)
    assert np.allclose(O.fwht(x), ref, atol=1e-5)
    # involution and norm preservation (reference tests/test_hadamard.py:19-33)
    assert np.allclose(O.fwht(O.fwht(x)), x, atol=1e-5)
    assert np.allclose(np.linalg.norm(O.fwht(x), axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


def test_fwht_rejects_non_power_of_two():
    with pytest.raises(ValueError, match="power of 2"):
        O.fwht(np.zeros((2, 100), np.float32))


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_codebook_matches_reference(golden, d, bits):
    b, l = O.lloyd_max_codebook(d, bits)
    assert np.array_equal(b, golden["codebooks"][f"b_{d}_{bits}"])
    assert np.array_equal(l, golden["codebooks"][f"l_{d}_{bits}"])
    # sorted and symmetric (reference tests/test_quantizer.py:12-25)
    assert np.all(np.diff(l) > 0)
    assert np.allclose(l, -l[::-1], atol=1e-3)


def test_quantize_is_bucketize_left():
    b = np.array([-1.0, -0.5, 0.0, 0.5, 1.0], np.float32)
    u = np.array([-2, -1, -0.75, -0.5, -0.25, 0.0, 0.25, 0.5, 0.75, 1.0, 2.0], np.float32)
    # torch.bucketize(right=False): #boundaries strictly below u; then -1, clamp [0, 3]
    want = [0, 0, 0, 0, 1, 1, 2, 2, 3, 3, 3]
    assert O.quantize(u, b, 2).tolist() == want


def test_pack3_every_group_brute_force():
    # all 8^2 combinations in two slots, random elsewhere, round trip + layout
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 8, (64, 8)).astype(np.uint8)
    codes[:, 2] = np.arange(64) % 8
    codes[:, 5] = np.arange(64) // 8
    p = O.pack(codes, 3)
    assert p.shape == (64, 3)
    assert np.array_equal(O.unpack(p, 3, 8), codes)
    w = p[:, 0].astype(np.uint32) | (p[:, 1].astype(np.uint32) << 8) | (p[:, 2].astype(np.uint32) << 16)
    for k in range(8):
        assert np.array_equal((w >> (3 * k)) & 7, codes[:, k])
    allb = np.arange(256 * 3, dtype=np.uint8).reshape(-1, 3)
    assert np.array_equal(O.pack(O.unpack(allb, 3, 8), 3), allb)


@pytest.mark.parametrize("bits", [1, 2, 4])
def test_pack_roundtrip_all_bytes(bits):
    allb = np.arange(256, dtype=np.uint8).reshape(-1, 8)
    d = 8 * 8 // bits
    assert np.array_equal(O.pack(O.unpack(allb, bits, d), bits), allb)
    if bits == 4:
        assert O.pack(np.array([[1, 2]], np.uint8), 4).tolist() == [[0x21]]
    if bits == 2:
        assert O.pack(np.array([[1, 2, 3, 0]], np.uint8), 2).tolist() == [[1 | 2 << 2 | 3 << 4]]


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_encode_decode_match_reference(golden, d, bits):
    enc, cb = golden["encode"], golden["codebooks"]
    key = f"{d}_{bits}"
    x = bf16_to_f32(enc["x_" + key])
    s = golden["signs"][f"s_{d}_42"]
    bnd = cb[f"b_{d}_{bits}"].astype(np.float32)
    lev = cb[f"l_{d}_{bits}"].astype(np.float32)
    p, n16, u, _ = O.encode(x, s, bnd, bits)
    assert np.array_equal(p, enc["packed_" + key])
    assert np.array_equal(n16.view(np.uint16), enc["norms_" + key])
    assert np.abs(u - enc["u_" + key]).max() < 1e-6
    dec = O.decode(enc["packed_" + key], enc["norms_" + key].view(np.float16), lev, s, bits, d)
    assert np.array_equal(dec, enc["dec_" + key])


def test_config1_4bit_outliers_match_reference(golden):
    enc, cb = golden["encode"], golden["codebooks"]
    x = bf16_to_f32(enc["x_cfg1"])
    s = golden["signs"]["s_128_0"]
    p, n16, _, _ = O.encode(x, s, cb["b_128_4"].astype(np.float32), 4)
    assert np.array_equal(p, enc["packed_cfg1"])
    assert np.array_equal(n16.view(np.uint16), enc["norms_cfg1"])
    dec = O.decode(p, n16, cb["l_128_4"].astype(np.float32), s, 4, 128)
    assert np.array_equal(dec, enc["dec_cfg1"])


def test_rotated_domain_score_identity():
    # <q, RHT^-1(c)> == <RHT(q), c> (the identity fused decode attention relies on;
    # reference tests/test_planar.py:132-185 checks it to 1e-3)
    rng = np.random.default_rng(1)
    d = 128
    s = np.where(rng.random(d) < 0.5, -1.0, 1.0).astype(np.float32)
    q = rng.standard_normal(d).astype(np.float32)
    c = rng.standard_normal((10, d)).astype(np.float32)
    lhs = O.inverse_rht(c, s).astype(np.float64) @ q.astype(np.float64)
    rhs = c.astype(np.float64) @ O.rht(q, s).astype(np.float64)
    assert np.allclose(lhs, rhs, atol=1e-4)


def test_lse_merge_equals_single_softmax():
    rng = np.random.default_rng(2)
    s = rng.standard_normal(40) * 3
    v = rng.standard_normal((40, 16))
    p = np.exp(s - s.max())
    full = (p / p.sum()) @ v
    parts_o, parts_l = [], []
    for a, b in ((0, 7), (7, 7), (7, 25), (25, 40)):
        if a == b:
            parts_o.append(np.zeros(16)); parts_l.append(-np.inf); continue
        ss = s[a:b]; m = ss.max(); pp = np.exp(ss - m)
        parts_o.append((pp / pp.sum()) @ v[a:b]); parts_l.append(m + np.log(pp.sum()))
    o, _ = O.lse_merge(np.array(parts_o), np.array(parts_l))
    assert np.allclose(o, full, atol=1e-12)


# ---- the torch restatement timed as bench.py's CPU baseline -----------------


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_torch_ref_matches_reference(golden, d, bits):
    """oracle/torch_ref.py reproduces the reference's unfused encode / decode
    outputs (tests/golden/encode.npz) byte for byte."""
    import torch
    from oracle import torch_ref as T
    enc, cb = golden["encode"], golden["codebooks"]
    key = f"{d}_{bits}"
    x = torch.from_numpy(enc["x_" + key].view(np.int16)).view(torch.bfloat16)
    s = torch.from_numpy(golden["signs"][f"s_{d}_42"])
    bnd = torch.from_numpy(cb[f"b_{d}_{bits}"].astype(np.float32))
    lev = torch.from_numpy(cb[f"l_{d}_{bits}"].astype(np.float32))
    p, n16 = T.encode(x, s, bnd, bits)
    assert np.array_equal(p.numpy(), enc["packed_" + key])
    assert np.array_equal(n16.view(torch.int16).numpy().view(np.uint16), enc["norms_" + key])
    dec = T.decode(p, n16, lev, s, bits, d)
    assert np.array_equal(dec.numpy(), enc["dec_" + key])


def test_torch_ref_config1_and_attention(golden):
    """Config-1 fixture (4-bit, outlier channels) byte for byte, and the dense
    attention against the numpy oracle's float64 attention."""
    import torch
    from oracle import torch_ref as T
    enc, cb = golden["encode"], golden["codebooks"]
    x = torch.from_numpy(enc["x_cfg1"].view(np.int16)).view(torch.bfloat16)
    s = torch.from_numpy(golden["signs"]["s_128_0"])
    p, n16 = T.encode(x, s, torch.from_numpy(cb["b_128_4"].astype(np.float32)), 4)
    assert np.array_equal(p.numpy(), enc["packed_cfg1"])
    assert np.array_equal(n16.view(torch.int16).numpy().view(np.uint16), enc["norms_cfg1"])
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 8, 128, generator=g)
    k = torch.randn(2, 2, 50, 128, generator=g)
    v = torch.randn(2, 2, 50, 128, generator=g)
    got = T.dense_attention(q, k, v, 128 ** -0.5).numpy()
    want = O.dense_decode_attention(q.numpy(), k.numpy(), v.numpy(), [50, 50], 128 ** -0.5)
    assert np.abs(got - want).max() < 1e-5


def test_tie_ulps_counts_float32_steps():
    """tie_ulps measures |u - cut| in float32 ulps of max(|cut|, d^-1/2)."""
    d = 128
    cuts = np.array([-0.2, 0.0, 0.15], np.float32)
    u = np.array([np.float32(0.15) + 3 * np.spacing(np.float32(0.15)),
                  np.float32(-0.2) - 2 * np.spacing(np.float32(0.2)),
                  5 * np.spacing(np.float32(d ** -0.5))], np.float64)
    assert np.allclose(O.tie_ulps(u, cuts, d), [3.0, 2.0, 5.0])
