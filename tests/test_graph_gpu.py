"""The library's launch paths under HIP graph capture (vLLM captures its decode
step; the reference keeps that path capturable, vllm_plugin/v1_backend.py:1165-1168).

Each case: one eager call first (one-time host set-up of the launch path), then
a torch CUDA graph of the same call with every tensor it touches allocated
before capture and held by the test.  The graph is replayed several times with
the program's own eager work and synchronisations between replays: new inputs
copied in place, an eager call into a second output, and each replay compared
with that eager result, bit for bit (same kernels, same inputs).
"""
import math

import pytest

import bench
import torch

pytestmark = pytest.mark.gpu


def _replay_check(cuda, refill, eager, graph_out, g, tag):
    for rep in range(3):
        refill(rep)
        torch.cuda.synchronize()
        want = eager()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = graph_out()
        assert torch.equal(got, want), f"{tag}: replay {rep} differs from eager"
        print(f"[graph {tag}] replay {rep} == eager", flush=True)


def _capture(fn):
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def test_encode_under_graph(cuda):
    from fused_turboquant import TurboQuantMSE
    tq = TurboQuantMSE(128, bits=3, seed=42, device=cuda)
    x = torch.randn(4099, 128, device=cuda).to(torch.bfloat16)
    holder = {}

    def enc():
        holder["g"] = tq.encode(x)  # allocates its outputs: from the graph's pool while capturing

    g = _capture(enc)
    ct_graph = holder["g"]  # the tensors the graph writes

    def refill(rep):
        x.copy_(torch.randn(4099, 128, device=cuda).to(torch.bfloat16) * (rep + 1))

    _replay_check(cuda, refill, lambda: tq.encode(x).indices, lambda: ct_graph.indices, g, "encode codes")


@pytest.mark.parametrize("splits", [1, 3])  # single-launch form, split form + merge launch
def test_paged_decode_under_graph(cuda, splits):
    from fused_turboquant import paged as P
    B, hq, hkv, d, ctx, page = 4, 16, 4, 128, 700, 16
    cache, q, bt, sl = bench.make_config3(cuda, B, hq, hkv, d, ctx, page)
    out_g = torch.empty(B, hq, d, dtype=torch.bfloat16, device=cuda)
    ws = torch.empty(P.workspace_bytes(B, hq, d, splits), dtype=torch.uint8, device=cuda)
    g = _capture(lambda: P.paged_decode_attention(q, cache.kv_cache, bt, sl, cache.k_quant, cache.v_quant,
                                                  num_splits=splits, out=out_g, workspace=ws))

    def refill(rep):
        q.copy_(torch.randn_like(q, dtype=torch.float32).to(q.dtype))
        sl.fill_(ctx - 37 * rep)

    def eager():
        return P.paged_decode_attention(q, cache.kv_cache, bt, sl, cache.k_quant, cache.v_quant, num_splits=splits)

    _replay_check(cuda, refill, eager, lambda: out_g, g, f"paged decode splits={splits}")


@pytest.mark.parametrize("splits", [1, 5])  # one launch writing the output itself, split form + merge launch
def test_v1_decode_under_graph(cuda, splits):
    from fused_turboquant import v1
    d, bs, hkv, hq, kb, vb = 128, 16, 4, 16, 4, 2
    layer = v1.TurboQuantV1Layer(d, kb, vb, v_rotate=True, device=cuda)
    B, L = 3, 900
    nb = B * ((L + bs - 1) // bs) + 2
    cache = torch.zeros(layer.kv_cache_shape(nb, bs, hkv), dtype=torch.uint8, device=cuda)
    slots = torch.randperm(nb * bs, device=cuda)[: B * L]
    layer.store(torch.randn(B * L, hkv, d, device=cuda).to(torch.bfloat16),
                torch.randn(B * L, hkv, d, device=cuda).to(torch.bfloat16), cache, slots)
    bt = (slots.view(B, L)[:, ::bs] // bs).to(torch.int32).contiguous()  # any page ids: values need not match
    sl = torch.full((B,), L, dtype=torch.int32, device=cuda)
    q = torch.randn(B, hq, d, device=cuda).to(torch.bfloat16)
    out_g = torch.empty(B, hq, d, dtype=torch.bfloat16, device=cuda)
    ws = torch.empty(v1.workspace_bytes(B, hq, d, splits), dtype=torch.uint8, device=cuda)
    g = _capture(lambda: layer.decode(q, cache, bt, sl, num_splits=splits, out=out_g, workspace=ws))

    def refill(rep):
        q.copy_(torch.randn_like(q, dtype=torch.float32).to(q.dtype))
        sl.fill_(L - 100 * rep)

    _replay_check(cuda, refill, lambda: layer.decode(q, cache, bt, sl, num_splits=splits), lambda: out_g, g,
                  f"v1 decode splits={splits}")


def test_raw_decode_under_graph(cuda):
    from fused_turboquant import raw
    d, bs, hkv, hq = 128, 16, 4, 16
    B, L = 3, 900
    nb = B * ((L + bs - 1) // bs) + 2
    cache = torch.zeros(nb, bs, hkv, 4 * d, dtype=torch.uint8, device=cuda)
    slots = torch.randperm(nb * bs, device=cuda)[: B * L]
    raw.raw_store(torch.randn(B * L, hkv, d, device=cuda).to(torch.bfloat16),
                  torch.randn(B * L, hkv, d, device=cuda).to(torch.bfloat16), cache, slots)
    bt = (slots.view(B, L)[:, ::bs] // bs).to(torch.int32).contiguous()
    sl = torch.full((B,), L, dtype=torch.int32, device=cuda)
    q = torch.randn(B, hq, d, device=cuda).to(torch.bfloat16)
    splits = 4
    out_g = torch.empty(B, hq, d, dtype=torch.float32, device=cuda)
    ws = torch.empty(raw.workspace_bytes(B, hq, d, splits), dtype=torch.uint8, device=cuda)
    scale = 1 / math.sqrt(d)
    g = _capture(lambda: raw.raw_decode_attention(q, cache, bt, sl, scale=scale, num_splits=splits, out=out_g,
                                                  workspace=ws))

    def refill(rep):
        q.copy_(torch.randn_like(q, dtype=torch.float32).to(q.dtype))
        sl.fill_(L - 100 * rep)

    def eager():
        return raw.raw_decode_attention(q, cache, bt, sl, scale=scale, num_splits=splits,
                                        out=torch.empty(B, hq, d, dtype=torch.float32, device=cuda))

    _replay_check(cuda, refill, eager, lambda: out_g, g, "raw decode")
