"""vLLM TURBOQUANT backend on gfx950, driven the way vLLM's v1 runner drives
it: ``do_kv_cache_update`` with the step's slot mapping, then ``forward`` with
the step's metadata (reference ``vllm_plugin/v1_backend.py:712-840``).

Expected values:
* decode tokens and continuation-chunk tokens: the oracle's float64 attention
  over the cache bytes the GPU store wrote, with the causal length of each
  query (cached + i + 1);
* fresh-prefill tokens: float64 causal attention over the raw bf16 K/V.
Tolerance: max abs error <= 2e-2 + 2^-8 |want|, mean <= 2e-3 max(1, mean |want|).
"""
import math
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu
D = 128


def _check(got, want, tag):
    err = np.abs(got.astype(np.float64) - want)
    bound = 2e-2 + 2.0 ** -8 * np.abs(want)
    mean_bound = 2e-3 * max(1.0, float(np.abs(want).mean()))
    print(f"[{tag}] max {err.max():.2e} mean {err.mean():.2e} worst/bound {(err / bound).max():.2f}", flush=True)
    assert (err <= bound).all() and err.mean() <= mean_bound, tag


def _causal_ref(q, k, v, scale, window=None):
    """float64 causal attention; q [n, Hq, d], k/v [n, Hkv, d] (the chunk is the whole sequence).
    With a window W, query i sees keys i - W + 1 .. i."""
    q, k, v = (np.asarray(t, np.float64) for t in (q, k, v))
    n, hq, d = q.shape
    G = hq // k.shape[1]
    out = np.zeros_like(q)
    for h in range(hq):
        s = q[:, h] @ k[:, h // G].T * scale
        s = s + np.triu(np.full((n, n), -np.inf), 1)
        if window is not None:
            s = s + np.tril(np.full((n, n), -np.inf), -window)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ v[:, h // G]
    return out


def _run_step(cuda, seqs, dtype_str, hq, hkv, vrot, monkeypatch, seed, bs=16, protect="0", lloyd=False,
              kind="rht", D=D, window=None):
    """seqs: list of (cached_len, query_len), decodes (query_len 1, cached > 0) first.
    Stores the cached tokens in earlier update calls, then runs one step.
    ``window``: the layer's sliding window (vLLM's ``sliding_window``)."""
    from fused_turboquant import vllm_plugin as vp
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", protect)
    monkeypatch.setenv("TURBOQUANT_V_ROTATE", "1" if vrot else "0")
    monkeypatch.setenv("TURBOQUANT_V_LLOYD_MAX", "1" if lloyd else "0")
    monkeypatch.setenv("TURBOQUANT_KIND", kind)
    g = torch.Generator().manual_seed(seed)
    Bk = vp.FusedTurboQuantV1Backend
    impl = vp.FusedTurboQuantV1Impl(hq, D, 1 / math.sqrt(D), hkv, kv_cache_dtype=dtype_str, sliding_window=window)
    layer = SimpleNamespace()
    pages = [(c + q + bs - 1) // bs for c, q in seqs]
    nb = sum(pages) + 5
    shape = Bk.get_kv_cache_shape(nb, bs, hkv, D, dtype_str)
    # boundary layers ("auto") get vLLM's bf16 allocation of the same shape
    cache = torch.zeros(shape, dtype=torch.bfloat16 if dtype_str == "auto" else torch.uint8, device=cuda)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    mb = max(pages)
    bt = torch.zeros(len(seqs), mb, dtype=torch.int32)
    used = 0
    full_k, full_v = [], []
    for i, (c, q) in enumerate(seqs):
        bt[i, :pages[i]] = perm[used:used + pages[i]]
        used += pages[i]
        k = torch.randn(c + q, hkv, D, generator=g).to(torch.bfloat16)
        v = torch.randn(c + q, hkv, D, generator=g).to(torch.bfloat16)
        full_k.append(k)
        full_v.append(v)

    def slots(i, lo, hi):
        pos = torch.arange(lo, hi)
        return bt[i].long()[pos // bs] * bs + pos % bs

    # earlier steps: the cached prefix of every sequence
    for i, (c, q) in enumerate(seqs):
        if c:
            impl.do_kv_cache_update(layer, full_k[i][:c].reshape(c, -1).to(cuda), full_v[i][:c].reshape(c, -1).to(cuda),
                                    cache, slots(i, 0, c).to(cuda))
    # this step's tokens
    qs = [torch.randn(q, hq, D, generator=g).to(torch.bfloat16) for _, q in seqs]
    key = torch.cat([full_k[i][c:] for i, (c, _) in enumerate(seqs)])
    val = torch.cat([full_v[i][c:] for i, (c, _) in enumerate(seqs)])
    query = torch.cat(qs)
    sm = torch.cat([slots(i, c, c + q) for i, (c, q) in enumerate(seqs)])
    N = query.shape[0]
    impl.do_kv_cache_update(layer, key.reshape(N, -1).to(cuda), val.reshape(N, -1).to(cuda), cache, sm.to(cuda))
    qlens = [q for _, q in seqs]
    qsl = torch.tensor([0] + np.cumsum(qlens).tolist(), dtype=torch.int32)
    nd = sum(1 for c, q in seqs if q == 1 and c > 0)
    md = SimpleNamespace(
        seq_lens=torch.tensor([c + q for c, q in seqs], dtype=torch.int32, device=cuda),
        block_table=bt.to(cuda), query_start_loc=qsl.to(cuda), slot_mapping=sm.to(cuda),
        num_actual_tokens=N, max_query_len=max(qlens), max_seq_len=max(c + q for c, q in seqs),
        is_prefill=nd < len(seqs), num_decodes=nd, num_decode_tokens=nd)
    output = torch.full((N, hq * D), float("nan"), dtype=torch.bfloat16, device=cuda)
    ret = impl.forward(layer, query.reshape(N, -1).to(cuda), key.reshape(N, -1).to(cuda),
                       val.reshape(N, -1).to(cuda), cache, md, output=output)
    torch.cuda.synchronize()
    assert ret is output
    got = output.float().cpu().numpy().reshape(N, hq, D)

    cache_np = cache.view(torch.uint8).cpu().numpy()
    raw = impl._is_raw
    cent = None if raw else layer._fused_tq_state.centroids.cpu().numpy()
    rot = None if raw or layer._fused_tq_state.rotation is None else layer._fused_tq_state.rotation.cpu().numpy()
    kb, vb = impl.key_bits, impl.value_bits
    for i, (c, q) in enumerate(seqs):
        a = int(qsl[i])
        if c == 0:
            want = _causal_ref(qs[i].float().numpy(), full_k[i].float().numpy(), full_v[i].float().numpy(),
                               1 / math.sqrt(D), window=window)
        else:
            sl = np.arange(c + 1, c + q + 1, dtype=np.int32)
            ks = None if window is None else np.maximum(sl - window, 0).astype(np.int32)
            btr = np.repeat(bt[i:i + 1].numpy(), q, axis=0)
            if raw:
                want = O.raw_decode_attention(qs[i].float().numpy(), cache_np, btr, sl, 1 / math.sqrt(D), kv_start=ks)
            else:
                want = O.v1_decode_attention(qs[i].float().numpy(), cache_np, btr, sl,
                                             None if impl.key_fp8 else cent, kb, vb,
                                             1 / math.sqrt(D), kv_start=ks, v_rotate=vrot or lloyd,
                                             v_lloyd_max=lloyd, rotation=rot, key_fp8=impl.key_fp8)
        kind = "prefill" if c == 0 else ("decode" if q == 1 else "continuation")
        _check(got[a:a + q], want, f"{dtype_str} vrot={vrot} W={window} seq{i} {kind} cached={c} q={q}")


@pytest.mark.parametrize("dtype_str,vrot", [("turboquant_3bit_nc", False), ("turboquant_k4v2_nc", True),
                                            ("turboquant_4bit_nc", True), ("turboquant_k3v4_nc", False)])
def test_decode_batch(cuda, monkeypatch, dtype_str, vrot):
    _run_step(cuda, [(1, 1), (100, 1), (513, 1), (4000, 1)], dtype_str, 32, 8, vrot, monkeypatch, seed=1)


@pytest.mark.parametrize("dtype_str,vrot", [("turboquant_3bit_nc", True), ("turboquant_k4v2_nc", False)])
def test_decode_batch_one_split(cuda, monkeypatch, dtype_str, vrot):
    """48 sequences x 8 kv heads: the Impl's split count is 1, where the decode
    kernel writes the output itself (no merge launch)."""
    from fused_turboquant import v1
    assert v1.default_splits(48, 8, 400) == 1
    seqs = [(1 + 7 * i, 1) for i in range(48)]
    _run_step(cuda, seqs, dtype_str, 32, 8, vrot, monkeypatch, seed=48)


def test_fresh_prefill_batch(cuda, monkeypatch):
    _run_step(cuda, [(0, 37), (0, 1), (0, 200)], "turboquant_3bit_nc", 16, 4, False, monkeypatch, seed=2)


def test_fresh_prefill_runs_of_equal_length(cuda, monkeypatch):
    """Consecutive fresh sequences of one length go through one batched SDPA
    launch with grouped K/V; runs of different lengths and a lone sequence
    between them stay separate.  Every row against float64 causal attention."""
    _run_step(cuda, [(0, 64), (0, 64), (0, 64), (0, 20), (0, 64), (0, 20), (0, 20)], "turboquant_3bit_nc", 32, 8,
              True, monkeypatch, seed=12)


@pytest.mark.parametrize("dtype_str,protect,d", [("turboquant_3bit_nc", "0", 128), ("turboquant_k4v2_nc", "0", 128),
                                                 ("turboquant_k3v4_nc", "0", 256), ("auto", "1", 128)])
def test_sliding_window_step(cuda, monkeypatch, dtype_str, protect, d):
    """A sliding-window layer (vLLM ``sliding_window=W``; reference
    v1_backend.py:299-318 accepts it): decode rows attend
    [max(0, seq_len - W), seq_len), continuation rows their own window, fresh
    prefill a banded causal mask.  Decodes longer and shorter than the window,
    a continuation chunk crossing it, fresh sequences longer than W.  Against
    the oracle's decode with kv_start and float64 banded causal attention."""
    _run_step(cuda, [(300, 1), (40, 1), (1000, 1), (200, 7), (0, 150), (0, 150), (0, 60)], dtype_str, 16, 4,
              dtype_str != "auto", monkeypatch, seed=13 + d, protect=protect, D=d, window=64)

def test_continuation_chunks(cuda, monkeypatch):
    _run_step(cuda, [(64, 17), (300, 64), (15, 2)], "turboquant_k4v2_nc", 8, 2, True, monkeypatch, seed=3)


def test_mixed_batch(cuda, monkeypatch):
    _run_step(cuda, [(40, 1), (2048, 1), (0, 33), (129, 9), (0, 1)], "turboquant_3bit_nc", 32, 8, True,
              monkeypatch, seed=4, bs=32, protect="1")


def test_no_metadata_zeroes_output(cuda):
    from fused_turboquant import vllm_plugin as vp
    impl = vp.FusedTurboQuantV1Impl(8, D, 0.1, 2, kv_cache_dtype="turboquant_3bit_nc")
    out = torch.ones(4, 8 * D, dtype=torch.bfloat16, device=cuda)
    cache = torch.zeros(2, 16, 2, 128, dtype=torch.uint8, device=cuda)
    q = torch.randn(4, 8 * D, device=cuda, dtype=torch.bfloat16)
    impl.forward(SimpleNamespace(), q, q[:, :2 * D], q[:, :2 * D], cache, None, output=out)
    assert not out.any()


@pytest.mark.parametrize("protect", ["1", "3", "8", "fp8"])
def test_boundary_layer_mixed_batch(cuda, monkeypatch, protect):
    """A boundary-protection layer (cache dtype "auto", vLLM's bf16 allocation):
    raw fp16 slots by default, 3-bit TurboQuant codes in the fp16-sized slot
    with TURBOQUANT_BOUNDARY_PROTECT=3; decode, fresh prefill and continuation."""
    _run_step(cuda, [(40, 1), (700, 1), (0, 33), (129, 9)], "auto", 32, 8, False, monkeypatch,
              seed=5, protect=protect)


@pytest.mark.parametrize("dtype_str,vrot", [("turboquant_k4v2_nc", False), ("turboquant_3bit_nc", True)])
def test_deferred_prefill_hybrid_decode(cuda, monkeypatch, dtype_str, vrot):
    """TURBOQUANT_DEFER_PREFILL=1 (reference v1_backend.py:673-686, 1095-1277),
    one sequence, as the reference supports it: a multi-token store goes to the
    fp16 prefix, single-token stores go to the slots, and a decode attends the
    prefix and the slots from position P on, merged by log-sum-exp.  First the
    seeded one-row zero prefix (no prefill deferred yet), then a 200-token
    deferred prefill followed by three decode steps.  Expected values: the
    oracle's float64 softmax over the union (fp16 prefix values, dequantised
    slot bytes the GPU wrote)."""
    from fused_turboquant import vllm_plugin as vp
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "0")
    monkeypatch.setenv("TURBOQUANT_V_ROTATE", "1" if vrot else "0")
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL", "1")
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL_CAPACITY", "256")
    hq, hkv, bs = 16, 4, 16
    g = torch.Generator().manual_seed(6)
    Bk = vp.FusedTurboQuantV1Backend
    impl = vp.FusedTurboQuantV1Impl(hq, D, 1 / math.sqrt(D), hkv, kv_cache_dtype=dtype_str)
    assert impl.defer_prefill and impl._prefix_capacity == 256
    layer = SimpleNamespace()
    nb = 20
    cache = torch.zeros(Bk.get_kv_cache_shape(nb, bs, hkv, D, dtype_str), dtype=torch.uint8, device=cuda)
    bt = torch.randperm(nb, generator=g).to(torch.int32)[None]
    kb, vb = impl.key_bits, impl.value_bits

    def slot(pos):
        return int(bt[0, pos // bs]) * bs + pos % bs

    def store1(pos, k, v):
        impl.do_kv_cache_update(layer, k.reshape(1, -1).to(cuda), v.reshape(1, -1).to(cuda), cache,
                                torch.tensor([slot(pos)], dtype=torch.int64, device=cuda))

    def decode(L, prefix_k, prefix_v, P, tag):
        q = torch.randn(1, hq, D, generator=g).to(torch.bfloat16)
        md = SimpleNamespace(seq_lens=torch.tensor([L], dtype=torch.int32, device=cuda), block_table=bt.to(cuda),
                             query_start_loc=torch.tensor([0, 1], dtype=torch.int32, device=cuda),
                             slot_mapping=None, num_actual_tokens=1, max_query_len=1, max_seq_len=L,
                             is_prefill=False, num_decodes=1, num_decode_tokens=1)
        out = torch.full((1, hq * D), float("nan"), dtype=torch.bfloat16, device=cuda)
        impl.forward(layer, q.reshape(1, -1).to(cuda), q.reshape(1, -1).to(cuda), q.reshape(1, -1).to(cuda),
                     cache, md, output=out)
        torch.cuda.synchronize()
        cent = layer._fused_tq_state.centroids.cpu().numpy()
        want = O.v1_hybrid_decode_attention(q.float().numpy(), prefix_k, prefix_v, P, cache.cpu().numpy(),
                                            bt.numpy(), np.array([L]), cent, kb, vb, 1 / math.sqrt(D),
                                            v_rotate=vrot)
        _check(out.float().cpu().numpy().reshape(1, hq, D), want, tag)

    # (1) no prefill deferred yet: the seeded prefix is one zero row, the slots start at 1
    for pos in range(9):
        store1(pos, torch.randn(hkv, D, generator=g).to(torch.bfloat16), torch.randn(hkv, D, generator=g).to(torch.bfloat16))
    zeros = np.zeros((1, hkv, D), np.float16)
    decode(9, zeros, zeros, 1, f"{dtype_str} seeded prefix")
    # (2) a 200-token prefill is deferred: fp16 prefix, nothing written to the slots
    P = 200
    kp = torch.randn(P, hkv, D, generator=g).to(torch.bfloat16)
    vp_ = torch.randn(P, hkv, D, generator=g).to(torch.bfloat16)
    before = cache.clone()
    impl.do_kv_cache_update(layer, kp.reshape(P, -1).to(cuda), vp_.reshape(P, -1).to(cuda), cache,
                            torch.tensor([slot(p) for p in range(P)], dtype=torch.int64, device=cuda))
    torch.cuda.synchronize()
    assert torch.equal(cache, before)
    pk, pv = kp.to(torch.float16).numpy(), vp_.to(torch.float16).numpy()
    for t in range(3):
        store1(P + t, torch.randn(hkv, D, generator=g).to(torch.bfloat16),
               torch.randn(hkv, D, generator=g).to(torch.bfloat16))
        decode(P + t + 1, pk, pv, P, f"{dtype_str} vrot={vrot} step {t}")


@pytest.mark.parametrize("dtype_str", ["turboquant_4bit_nc", "turboquant_k3v4_nc", "turboquant_k4v2_nc"])
def test_v_lloyd_max_step(cuda, monkeypatch, dtype_str):
    """TURBOQUANT_V_LLOYD_MAX=1 through the Impl (reference v1_backend.py:728-740,
    1086-1092): 4-bit V stores Lloyd-Max codes and decodes them with the norm
    correction; 2-bit V (K4V2) stays uniform but rotated.  Decode, fresh
    prefill and continuation in one mixed step."""
    _run_step(cuda, [(40, 1), (700, 1), (0, 33), (129, 9)], dtype_str, 32, 8, False, monkeypatch,
              seed=7, lloyd=True)


@pytest.mark.parametrize("vrot", [False, True])
def test_planar_kind_step(cuda, monkeypatch, vrot):
    """TURBOQUANT_KIND=planar through the Impl (reference v1_backend.py:516-523,
    rotation/planar.py): the store, decode and merge kernels rotate by the
    planar matrix.  Decode, fresh prefill and continuation in one mixed step,
    against the oracle with the same matrix."""
    _run_step(cuda, [(40, 1), (700, 1), (0, 33), (129, 9)], "turboquant_k4v2_nc", 32, 8, vrot, monkeypatch,
              seed=11, kind="planar")


@pytest.mark.parametrize("defer", [False, True])
def test_impl_decode_under_graph_capture(cuda, monkeypatch, defer):
    """A decode-only step of FusedTurboQuantV1Impl.forward captured in a HIP
    graph (per-layer scratch, output written in place, the split count fixed
    at TURBOQUANT_MAX_KV_SPLITS): three replays with new queries, an eager step
    between them, each replay bit-identical to the eager forward of the same
    inputs (the eager step picks the same split count here)."""
    from fused_turboquant import vllm_plugin as vp
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "0")
    monkeypatch.setenv("TURBOQUANT_V_ROTATE", "1")
    monkeypatch.setenv("TURBOQUANT_V_LLOYD_MAX", "0")
    monkeypatch.setenv("TURBOQUANT_KIND", "rht")
    monkeypatch.setenv("TURBOQUANT_MAX_KV_SPLITS", "4")
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL", "1" if defer else "0")
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL_CAPACITY", "256")
    hq, hkv, bs = 8, 2, 16
    lens = [8100, 8192, 7000]
    B = len(lens)
    impl = vp.FusedTurboQuantV1Impl(hq, D, 1 / math.sqrt(D), hkv, kv_cache_dtype="turboquant_k4v2_nc")
    layer = SimpleNamespace()
    g = torch.Generator().manual_seed(77)
    pages = [(n + bs - 1) // bs for n in lens]
    nb = sum(pages)
    cache = torch.zeros(vp.FusedTurboQuantV1Backend.get_kv_cache_shape(nb, bs, hkv, D, "turboquant_k4v2_nc"),
                        dtype=torch.uint8, device=cuda)
    perm = torch.randperm(nb, generator=g).to(torch.int32)
    bt = torch.zeros(B, max(pages), dtype=torch.int32)
    used = 0
    for i, n in enumerate(lens):
        bt[i, :pages[i]] = perm[used:used + pages[i]]
        used += pages[i]
        k = torch.randn(n, hkv * D, generator=g).to(torch.bfloat16).to(cuda)
        v = torch.randn(n, hkv * D, generator=g).to(torch.bfloat16).to(cuda)
        pos = torch.arange(n)
        impl.do_kv_cache_update(layer, k, v, cache, (bt[i].long()[pos // bs] * bs + pos % bs).to(cuda))
    md = SimpleNamespace(seq_lens=torch.tensor(lens, dtype=torch.int32, device=cuda), block_table=bt.to(cuda),
                         query_start_loc=torch.arange(B + 1, dtype=torch.int32, device=cuda), num_actual_tokens=B,
                         max_query_len=1, max_seq_len=max(lens), is_prefill=False, num_decodes=B,
                         num_decode_tokens=B)
    q = torch.empty(B, hq * D, dtype=torch.bfloat16, device=cuda)
    kv = torch.zeros(B, hkv * D, dtype=torch.bfloat16, device=cuda)
    out_g = torch.empty(B, hq * D, dtype=torch.bfloat16, device=cuda)

    def new_q(rep):
        q.copy_(torch.randn(B, hq * D, generator=torch.Generator().manual_seed(100 + rep)).to(torch.bfloat16))

    new_q(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up: per-layer scratch allocated before the capture
        impl.forward(layer, q, kv, kv, cache, md, output=out_g)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        impl.forward(layer, q, kv, kv, cache, md, output=out_g)
    for rep in range(1, 4):
        new_q(rep)
        graph.replay()
        torch.cuda.synchronize()
        got = out_g.clone()
        want = impl.forward(layer, q, kv, kv, cache, md, output=torch.empty_like(out_g))
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), rep


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("dtype_str,protect", [("turboquant_3bit_nc", "0"), ("turboquant_k4v2_nc", "0"),
                                               ("auto", "1"), ("auto", "fp8")])
def test_head_sizes_64_256(cuda, monkeypatch, d, dtype_str, protect):
    """Head sizes 64 and 256 (the fp32 decode kernel; raw fp16 boundary slots
    likewise): decode, fresh prefill and continuation in one step."""
    _run_step(cuda, [(40, 1), (700, 1), (0, 21), (129, 9)], dtype_str, 16, 4, d == 256, monkeypatch,
              seed=d + len(dtype_str), protect=protect, D=d)


@pytest.mark.parametrize("dtype_str", ["turboquant_k1v2_nc", "turboquant_k4v1_nc", "turboquant_k1v1_nc"])
def test_one_bit_aliases(cuda, monkeypatch, dtype_str):
    """The 1-bit turboquant_k{K}v{V}_nc aliases (reference plugin.py:322): the
    host preset's slot, 1-bit codes, decode on the fp32 kernel."""
    _run_step(cuda, [(64, 1), (900, 1), (33, 5)], dtype_str, 32, 8, True, monkeypatch, seed=9)
