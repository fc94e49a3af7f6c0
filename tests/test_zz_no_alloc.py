"""Allocation-free v1 decode attention (ftq_v1_decode_attention_noalloc)
against the workspace entry point (ftq_v1_decode_attention) through the C ABI.

Both run the same kernels; the first takes its split-K partials in a device
array of the library instead of a caller's workspace, so the outputs must be
bit-identical.  Two calls in a row, the second on a smaller input, show that
what the first call left in the shared array does not leak into the second.
"""
import ctypes
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _bind_noalloc(L):
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    L.ftq_v1_decode_attention_noalloc.argtypes = [
        vp, i32, vp, i64, i32, i64, i64, i64, vp, i32, vp, vp, i32, i32, i32, i32, vp, i32, i32,
        f32, i32, i32, vp, i32, vp]
    L.ftq_v1_decode_attention_noalloc.restype = ctypes.c_int
    L.ftq_v1_scratch_bytes.argtypes = []
    L.ftq_v1_scratch_bytes.restype = ctypes.c_int64
    return L


def _case(dev, seed, B, hq, hkv, lens, kb, vb, vrot):
    from fused_turboquant import v1
    d, bs = 128, 16
    g = torch.Generator().manual_seed(seed)
    layer = v1.TurboQuantV1Layer(d, kb, vb, v_rotate=vrot, device=dev)
    pages = [(n + bs - 1) // bs for n in lens]
    nb = sum(pages) + 2
    cache = torch.zeros(layer.kv_cache_shape(nb, bs, hkv), dtype=torch.uint8, device=dev)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.zeros(B, max(pages), dtype=torch.int32)
    used = 0
    for b, n in enumerate(lens):
        bt[b, :pages[b]] = perm[used:used + pages[b]]
        used += pages[b]
        k = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).to(dev)
        v = torch.randn(n, hkv, d, generator=g).to(torch.bfloat16).to(dev)
        pos = torch.arange(n)
        slots = (bt[b, pos // bs].long() * bs + pos % bs).to(dev)
        layer.store(k, v, cache, slots)
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16).to(dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    return layer, cache, q, bt.to(dev), sl


def _run_both(L, dev, layer, cache, q, bt, sl, splits):
    from fused_turboquant import _lib, v1
    B, hq, d = q.shape
    nb, bs, hkv, _ = cache.shape
    sb, sp, sh = cache.stride(0), cache.stride(1), cache.stride(2)
    scale = 1.0 / math.sqrt(d)
    flags = 1 if layer.v_rotate else 0
    ref = torch.full((B, hq, d), float("nan"), dtype=torch.bfloat16, device=dev)
    ws = torch.empty(v1.workspace_bytes(B, hq, d, splits), dtype=torch.uint8, device=dev)
    st = _lib.stream_ptr(dev)
    common = (q.data_ptr(), _lib.BF16, cache.data_ptr(), nb, bs, sb, sp, sh, bt.data_ptr(), bt.shape[1],
              sl.data_ptr(), None, B, hq, hkv, d, layer.centroids.data_ptr(), layer.key_bits,
              layer.value_bits, scale, flags, splits)
    _lib.check(v1._bind().ftq_v1_decode_attention(*common, ws.data_ptr(), ws.numel(), ref.data_ptr(),
                                                  _lib.BF16, st))
    got = torch.full((B, hq, d), float("nan"), dtype=torch.bfloat16, device=dev)
    _lib.check(L.ftq_v1_decode_attention_noalloc(*common, got.data_ptr(), _lib.BF16, st))
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_matches_workspace_entry_point_twice(cuda):
    from fused_turboquant import _lib, v1
    L = _bind_noalloc(v1._bind())
    assert L.ftq_v1_scratch_bytes() == 16 << 20
    # first call: 3 sequences, GQA 4, 16 splits
    big = _case(cuda, 1, 3, 16, 4, [1500, 700, 2049], 4, 2, True)
    ref1, got1 = _run_both(L, cuda, *big, splits=16)
    assert not torch.isnan(ref1.float()).any()
    assert torch.equal(got1, ref1)
    # second call, smaller: 1 sequence, GQA 2, 3 splits; the first call's
    # partials are still in the scratch array
    small = _case(cuda, 2, 1, 4, 2, [333], 3, 3, False)
    ref2, got2 = _run_both(L, cuda, *small, splits=3)
    assert not torch.isnan(ref2.float()).any()
    assert torch.equal(got2, ref2)
    # the first result again, after the second call
    _, got1b = _run_both(L, cuda, *big, splits=16)
    assert torch.equal(got1b, ref1)


def test_noalloc_rejects_shapes_beyond_the_scratch(cuda):
    from fused_turboquant import _lib, v1
    L = _bind_noalloc(v1._bind())
    layer, cache, q, bt, sl = _case(cuda, 3, 1, 4, 2, [64], 4, 2, False)
    B, hq, d = q.shape
    nb, bs, hkv, _ = cache.shape
    # 64 * 32 * 1024 * 129 * 4 bytes of partials > 16 MiB (an otherwise valid
    # shape: GQA 16): rejected before any launch
    out = torch.empty(64, 32, d, dtype=torch.bfloat16, device=cuda)
    rc = L.ftq_v1_decode_attention_noalloc(
        q.data_ptr(), _lib.BF16, cache.data_ptr(), nb, bs, cache.stride(0), cache.stride(1), cache.stride(2),
        bt.data_ptr(), bt.shape[1], sl.data_ptr(), None, 64, 32, hkv, d, layer.centroids.data_ptr(),
        4, 2, 0.088, 0, 1024, out.data_ptr(), _lib.BF16, _lib.stream_ptr(cuda))
    assert rc == -1
    assert b"16 MiB" in L.ftq_last_error()
