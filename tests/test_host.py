"""Host-side logic and the C ABI surface, without a GPU."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest
import torch

from conftest import ROOT


def _built_lib():
    from fused_turboquant import _lib
    if not os.path.exists(_lib.LIB_PATH):
        import __graft_entry__
        __graft_entry__.build()
    return _lib


def _declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        txt = open(h).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        names |= set(re.findall(r"\b(ftq_\w+)\s*\(", txt))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared_symbols()
    for must in ("ftq_encode", "ftq_decode", "ftq_rht", "ftq_last_error", "ftq_version"):
        assert must in names


def test_library_exports_every_declared_symbol():
    L = _built_lib().lib()
    for name in _declared_symbols():
        assert hasattr(L, name), f"{name} declared in include/ but not exported"
    assert L.ftq_version() == 1


def test_argument_errors_raise_without_touching_the_gpu():
    _lib = _built_lib()
    L = _lib.lib()
    rc = L.ftq_encode(None, 2, 4, 100, None, None, 3, None, None, None)
    assert rc == -1 and b"head_dim" in L.ftq_last_error()
    rc = L.ftq_encode(None, 2, 4, 128, None, None, 5, None, None, None)
    assert rc == -1 and b"bits" in L.ftq_last_error()
    with pytest.raises(ValueError, match="head_dim"):
        _lib.check(L.ftq_decode(None, None, 4, 96, None, None, 3, None, 0, None))
    assert L.ftq_encode(None, 2, 0, 128, None, None, 3, None, None, None) == 0  # empty input


def _c_class(L, b, bits):
    b = np.ascontiguousarray(b, dtype=np.float32)
    return L.ftq_codebook_class(b.ctypes.data_as(ctypes.c_void_p), bits)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_codebook_class_host_and_c_agree(bits):
    """The encoder's symmetric kernel is chosen from the codebook class; the
    Python rule and the C ABI's must agree, and the library codebooks of
    d = 64 / 128 are symmetric in fp32 while those of d = 256 are not."""
    from fused_turboquant.core.lloyd_max import CB_ANY, CB_SYMMETRIC, codebook_class, compute_lloyd_max_codebook
    L = _built_lib().lib()
    for d, want in ((64, CB_SYMMETRIC), (128, CB_SYMMETRIC), (256, CB_ANY)):
        b = compute_lloyd_max_codebook(d, bits)[0].astype(np.float32)
        assert codebook_class(b, bits) == want == _c_class(L, b, bits), (d, bits)
    mid = 1 << (bits - 1)
    pos = np.sort(np.random.default_rng(bits).uniform(0.01, 0.3, mid - 1)).astype(np.float32)
    sym = np.concatenate([[-1.0], -pos[::-1], [0.0], pos, [1.0]]).astype(np.float32)
    cases = {"symmetric": (sym, CB_SYMMETRIC)}
    tilt = sym.copy()
    tilt[mid + 1] = np.nextafter(tilt[mid + 1], np.float32(1))  # one ulp off
    cases["one ulp asymmetric"] = (tilt, CB_ANY)
    wide = sym.copy()
    wide[mid] = sym[mid + 1] * 1.5  # middle beyond the first positive boundary
    cases["middle too wide"] = (np.sort(wide), CB_ANY)
    uns = sym.copy()
    uns[1], uns[2] = uns[2], uns[1]
    cases["unsorted"] = (uns, CB_ANY)
    nan = sym.copy()
    nan[mid] = np.nan
    cases["nan"] = (nan, CB_ANY)
    for name, (b, want) in cases.items():
        assert codebook_class(b, bits) == want == _c_class(L, b, bits), name
    assert _c_class(L, sym, 5) == -1 and b"bits" in L.ftq_last_error()


def test_encode_cb_rejects_unknown_class():
    L = _built_lib().lib()
    rc = L.ftq_encode_cb(None, 2, 4, 128, None, None, 3, 7, None, None, None)
    assert rc == -1 and b"codebook_class" in L.ftq_last_error()


def test_encode_kv_validates_before_launch():
    """ftq_encode_kv's argument checks run on the host (no device needed)."""
    L = _built_lib().lib()
    assert L.ftq_encode_kv(None, None, 2, 4, 128, None, None, 3, 7, None, None, None, None, None) == -1
    assert b"codebook_class" in L.ftq_last_error()
    assert L.ftq_encode_kv(None, None, 2, 4, 96, None, None, 3, 0, None, None, None, None, None) == -1
    assert b"head_dim" in L.ftq_last_error()
    assert L.ftq_encode_kv(None, None, 2, 4, 128, None, None, 3, 0, None, None, None, None, None) == -1
    assert b"null" in L.ftq_last_error()
    assert L.ftq_encode_kv(None, None, 2, 0, 128, None, None, 3, 0, None, None, None, None, None) == 0


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_product_codebook_matches_reference(golden, d, bits):
    from fused_turboquant.core.lloyd_max import compute_lloyd_max_codebook
    b, l = compute_lloyd_max_codebook(d, bits)
    assert np.array_equal(b, golden["codebooks"][f"b_{d}_{bits}"])
    assert np.array_equal(l, golden["codebooks"][f"l_{d}_{bits}"])


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("seed", [0, 1, 42])
def test_signs_match_reference(golden, d, seed):
    from fused_turboquant.core.hadamard import generate_rht_signs
    assert np.array_equal(generate_rht_signs(d, seed).numpy(), golden["signs"][f"s_{d}_{seed}"])


def test_cpu_tensors_are_rejected():
    from fused_turboquant import TurboQuantMSE
    from fused_turboquant._lib import FusedTQError
    tq = TurboQuantMSE(128, bits=3)
    with pytest.raises(FusedTQError, match="ROCm"):
        tq.encode(torch.zeros(4, 128))


def test_quantizer_validation():
    from fused_turboquant import TurboQuantMSE
    with pytest.raises(ValueError, match="power of 2"):
        TurboQuantMSE(100)
    with pytest.raises(ValueError, match="bits"):
        TurboQuantMSE(128, bits=5)


def test_torch_packers_match_oracle():
    from fused_turboquant.core import packing as P
    from oracle import tq_oracle as O
    rng = np.random.default_rng(0)
    for bits, pk, up in ((4, P.pack_nibbles, P.unpack_nibbles), (3, P.pack_3bit, P.unpack_3bit),
                         (2, P.pack_2bit, P.unpack_2bit)):
        c = rng.integers(0, 1 << bits, (7, 128)).astype(np.uint8)
        p = pk(torch.from_numpy(c)).numpy()
        assert np.array_equal(p, O.pack(c, bits))
        assert np.array_equal(up(torch.from_numpy(p), 128).numpy(), c)


def test_paged_choose_splits_host_heuristic():
    """ftq_paged_choose_splits: 1 (the single-launch form) only for d = 128,
    GQA group <= 4 and batch * Hkv filling 256 CUs in rounds at least 3/4 full;
    otherwise the split form's default."""
    from fused_turboquant import paged as P
    L = P._bind()
    dflt = L.ftq_paged_default_splits
    assert P.default_splits(32, 8, 8192, 32, 128) == 1       # B 32 x 8 kv heads: 256 workgroups
    assert P.default_splits(64, 8, 8192, 32, 128) == 1       # two full rounds
    assert P.default_splits(48, 8, 8192, 32, 128) == 1       # 384 of 512 slots: 3/4
    assert P.default_splits(40, 8, 8192, 32, 128) == dflt(40, 8, 8192)  # 320 of 512: below 3/4
    assert P.default_splits(16, 8, 8192, 32, 128) == dflt(16, 8, 8192)  # 128 workgroups: too few
    assert P.default_splits(32, 8, 8192, 64, 128) == dflt(32, 8, 8192)  # GQA 8
    assert P.default_splits(32, 8, 8192, 32, 256) == dflt(32, 8, 8192)  # d = 256
    assert P.default_splits(32, 8, 8192) == dflt(32, 8, 8192)           # geometry unknown
