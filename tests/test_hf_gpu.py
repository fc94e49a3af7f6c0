"""HF integration on gfx950: the patched model's decode runs the paged decode
kernel over codes stored by the paged store kernel.

* cache level: decode_attention == float64 softmax attention over the oracle's
  decode of the stored codes (bf16 tolerance, as for the paged kernel);
* model level: a left-padded batch gives each sequence the logits it gets
  alone (padding is not stored); patched vs unpatched first decode logits
  agree to quantisation accuracy; K-only layers and unpatch work.
"""
import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O

pytestmark = pytest.mark.gpu


def _tiny_llama(cuda, layers=2, heads=4, kv_heads=2, head_dim=128):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=heads * head_dim, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=head_dim,
                      vocab_size=320, max_position_embeddings=512)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(device=cuda, dtype=torch.bfloat16).eval()


@pytest.mark.parametrize("bk,bv", [(3, 3), (4, 2)])
def test_cache_decode_attention_matches_dense(cuda, bk, bv):
    from fused_turboquant import TurboQuantMSE
    from fused_turboquant.hf import CompressedKVCache
    g = torch.Generator(device="cpu").manual_seed(bk * 10 + bv)
    B, hkv, hq, d = 3, 2, 8, 128
    k_tq, v_tq = TurboQuantMSE(d, bits=bk, device=cuda), TurboQuantMSE(d, bits=bv, device=cuda)
    cache = CompressedKVCache(k_tq)
    cache.set_layer_quantizer(0, k_tq)
    cache.set_layer_quantizer_v(0, v_tq)
    # prefill of 37 tokens with the first 5 of sequence 0 masked out, then 40 decode steps
    k = torch.randn(B, hkv, 37, d, generator=g).to(torch.bfloat16).to(cuda)
    v = torch.randn(B, hkv, 37, d, generator=g).to(torch.bfloat16).to(cuda)
    keep = torch.ones(B, 37, dtype=torch.bool, device=cuda)
    keep[0, :5] = False
    cache.store_compressed_kv(k, v, 0, keep=keep)
    for _ in range(40):
        cache.store_compressed_kv(torch.randn(B, hkv, 1, d, generator=g).to(torch.bfloat16).to(cuda),
                                  torch.randn(B, hkv, 1, d, generator=g).to(torch.bfloat16).to(cuda), 0)
    assert cache.seq_lens(0) == [72, 77, 77]
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16)
    out = cache.decode_attention(q.to(cuda), 0, 1 / math.sqrt(d)).float().cpu().numpy()
    ke, ve = cache.get_compressed_key(0), cache.get_compressed_value(0)
    S = ke["packed_indices"].shape[2]
    kd = O.decode(ke["packed_indices"].cpu().numpy().reshape(-1, d * bk // 8), ke["norms"].cpu().numpy().reshape(-1),
                  k_tq.quantizer.levels.cpu().numpy(), k_tq.rotation.signs.cpu().numpy(), bk, d).reshape(B, hkv, S, d)
    vd = O.decode(ve["packed_indices"].cpu().numpy().reshape(-1, d * bv // 8), ve["norms"].cpu().numpy().reshape(-1),
                  v_tq.quantizer.levels.cpu().numpy(), v_tq.rotation.signs.cpu().numpy(), bv, d).reshape(B, hkv, S, d)
    want = O.dense_decode_attention(q.float().numpy(), kd, vd, cache.seq_lens(0), 1 / math.sqrt(d))
    err = np.abs(out - want)
    print(f"[hf cache K{bk}V{bv}] max {err.max():.2e} mean {err.mean():.2e}")
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
    # the decoded cache reproduces the stored vectors to quantisation accuracy
    vv = v[1].float().cpu().numpy()  # sequence 1 stored all 37 prefill tokens
    cos = (vd[1, :, :37] * vv).sum(-1) / np.linalg.norm(vd[1, :, :37], axis=-1) / np.linalg.norm(vv, axis=-1)
    assert cos.mean() > (0.97 if bv >= 3 else 0.9)


def _gen(model, ids, mask, cache, n):
    out = model.generate(input_ids=ids, attention_mask=mask, past_key_values=cache, max_new_tokens=n,
                         do_sample=False, output_logits=True, return_dict_in_generate=True, pad_token_id=0)
    return out.sequences, torch.stack(out.logits, 1).float()


def test_padded_batch_matches_single_sequences(cuda):
    from fused_turboquant.hf import patch_model
    model = _tiny_llama(cuda)
    cache = patch_model(model, bits=4, verify=True)
    g = torch.Generator().manual_seed(5)
    a = torch.randint(1, 320, (1, 5), generator=g)
    b = torch.randint(1, 320, (1, 9), generator=g)
    ids = torch.zeros(2, 9, dtype=torch.long)
    mask = torch.zeros(2, 9, dtype=torch.long)
    ids[0, 4:], mask[0, 4:] = a[0], 1
    ids[1], mask[1] = b[0], 1
    with torch.inference_mode():
        _, lb = _gen(model, ids.to(cuda), mask.to(cuda), cache, 4)
        cache.reset()
        _, la = _gen(model, a.to(cuda), torch.ones_like(a).to(cuda), cache, 4)
        cache.reset()
        _, l1 = _gen(model, b.to(cuda), torch.ones_like(b).to(cuda), cache, 4)
        cache.reset()
    for got, want, tag in ((lb[0], la[0], "seq a"), (lb[1], l1[0], "seq b")):
        diff = (got - want).abs().max().item()
        print(f"[hf padded batch {tag}] max logit diff {diff:.3e} (|logit| max {want.abs().max().item():.2f})")
        assert diff <= 2e-2 * max(1.0, want.abs().max().item())


def test_patched_logits_close_to_unpatched(cuda):
    from fused_turboquant.hf import patch_model, unpatch_model
    model = _tiny_llama(cuda)
    ids = torch.randint(1, 320, (2, 24), generator=torch.Generator().manual_seed(9)).to(cuda)
    mask = torch.ones_like(ids)
    with torch.inference_mode():
        _, ref = _gen(model, ids, mask, None, 3)
        cache = patch_model(model, bits=4, verify=False)
        _, got = _gen(model, ids, mask, cache, 3)
        unpatch_model(model)
        _, again = _gen(model, ids, mask, None, 3)
    # step 0 comes from the prefill (full precision in both), later steps read the 4-bit cache
    assert torch.allclose(got[:, 0], ref[:, 0], atol=1e-2, rtol=1e-2)
    cos = torch.nn.functional.cosine_similarity(got[:, 1:].reshape(-1, got.shape[-1]), ref[:, 1:].reshape(-1, ref.shape[-1]), dim=-1)
    print(f"[hf patched vs unpatched] decode logits cos min {cos.min().item():.4f}")
    assert cos.min() > 0.98
    assert torch.equal(again, ref)


@pytest.mark.parametrize("compress_v", [False, "boundary"])
def test_k_only_layers(cuda, compress_v):
    from fused_turboquant.hf import patch_model
    model = _tiny_llama(cuda, layers=4)
    ids = torch.randint(1, 320, (2, 12), generator=torch.Generator().manual_seed(3)).to(cuda)
    with torch.inference_mode():
        _, ref = _gen(model, ids, torch.ones_like(ids), None, 3)
        cache = patch_model(model, bits=4, compress_v=compress_v, verify=False)
        _, got = _gen(model, ids, torch.ones_like(ids), cache, 3)
    cos = torch.nn.functional.cosine_similarity(got.reshape(-1, got.shape[-1]), ref.reshape(-1, ref.shape[-1]), dim=-1)
    assert torch.isfinite(got).all() and cos.min() > 0.98, cos.min()


def test_padded_batch_continuation_chunk(cuda):
    """A left-padded batch prefilled, then a 3-token chunk of new tokens per
    sequence (a multi-token continuation over the compressed past), against
    each sequence run alone through the same steps."""
    from fused_turboquant.hf import patch_model
    model = _tiny_llama(cuda)
    cache = patch_model(model, bits=4, verify=False)
    g = torch.Generator().manual_seed(8)
    a = torch.randint(1, 320, (1, 4), generator=g)
    b = torch.randint(1, 320, (1, 10), generator=g)
    ca = torch.randint(1, 320, (1, 3), generator=g)
    cb = torch.randint(1, 320, (1, 3), generator=g)
    ids = torch.zeros(2, 10, dtype=torch.long)
    mask = torch.zeros(2, 10, dtype=torch.long)
    ids[0, 6:], mask[0, 6:] = a[0], 1
    ids[1], mask[1] = b[0], 1

    def two_steps(p_ids, p_mask, c_ids):
        # positions counted over each sequence's real tokens (as generate() does), so a
        # left-padded sequence's keys are rotated exactly as when it runs alone
        pos = (p_mask.cumsum(-1) - 1).clamp(min=0)
        cpos = p_mask.sum(-1, keepdim=True) + torch.arange(c_ids.shape[1])[None]
        with torch.inference_mode():
            model(input_ids=p_ids.to(cuda), attention_mask=p_mask.to(cuda), position_ids=pos.to(cuda),
                  past_key_values=cache, use_cache=True)
            m2 = torch.cat([p_mask, torch.ones(p_mask.shape[0], c_ids.shape[1], dtype=torch.long)], 1)
            out = model(input_ids=c_ids.to(cuda), attention_mask=m2.to(cuda), position_ids=cpos.to(cuda),
                        past_key_values=cache, use_cache=True)
        cache.reset()
        return out.logits.float()

    lb = two_steps(ids, mask, torch.cat([ca, cb], 0))
    la = two_steps(a, torch.ones_like(a), ca)
    l1 = two_steps(b, torch.ones_like(b), cb)
    for got, want, tag in ((lb[0], la[0], "seq a"), (lb[1], l1[0], "seq b")):
        diff = (got - want).abs().max().item()
        print(f"[hf padded continuation {tag}] max logit diff {diff:.3e} (|logit| max {want.abs().max().item():.2f})")
        assert diff <= 2e-2 * max(1.0, want.abs().max().item())


def _tiny_gemma4(cuda, window=8, sinks=0):
    """A random-init Gemma 4 text model: sliding layers at head_dim 64 (flat
    rows, window attention), full layers at head_dim 128 with K = V (no
    v_proj) and one kv head (paged decode), scaling 1.0, q/k/v norms."""
    from transformers import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM
    cfg = Gemma4TextConfig(vocab_size=320, hidden_size=256, intermediate_size=512, num_hidden_layers=4,
                           num_attention_heads=4, num_key_value_heads=2, head_dim=64, global_head_dim=128,
                           sliding_window=window,
                           layer_types=["sliding_attention", "full_attention", "sliding_attention", "full_attention"],
                           attention_k_eq_v=True, num_global_key_value_heads=1, vocab_size_per_layer_input=320,
                           hidden_size_per_layer_input=16, max_position_embeddings=512)
    cfg.sink_tokens = sinks
    torch.manual_seed(0)
    model = Gemma4ForCausalLM(cfg)
    # Gemma scores with scaling 1.0 over RMS-normalised q and k: at random init
    # (norm weights 1) the scores have std sqrt(head_dim) and every softmax is
    # near one-hot, so any K error flips it.  Trained models are far smoother;
    # shrinking the query norm weights gives this one softmaxes of that kind.
    with torch.no_grad():
        for n, mod in model.named_modules():
            if n.endswith("self_attn"):
                mod.q_norm.weight.mul_(0.1)
    return model.to(device=cuda, dtype=torch.bfloat16).eval()


def _teacher_forced(model, ids, steps, cache):
    """Logits of a prompt prefill and then of each token of `steps` fed one at a time."""
    out = [model(ids, past_key_values=cache, use_cache=True).logits[:, -1].float()]
    for t in range(steps.shape[1]):
        out.append(model(steps[:, t:t + 1], past_key_values=cache, use_cache=True).logits[:, -1].float())
    return torch.stack(out, 1)


def test_gemma4_patched_close_to_unpatched(cuda):
    """Gemma 4 (per-layer head dims, K = V layers, sliding windows shorter than
    the prompt): fed the same tokens, the patched model's decode logits follow
    the unpatched model's to quantisation accuracy, and unpatching restores it
    exactly."""
    from transformers import DynamicCache
    from fused_turboquant.hf import check_model_compatibility, patch_model, unpatch_model
    model = _tiny_gemma4(cuda)
    rep = check_model_compatibility(model)
    assert rep["compatible"] and rep["head_dims"] == [64, 128] and rep["k_eq_v_layers"] == 2, rep
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(1, 320, (1, 30), generator=g).to(cuda)
    steps = torch.randint(1, 320, (1, 12), generator=g).to(cuda)
    with torch.inference_mode():
        ref = _teacher_forced(model, ids, steps, DynamicCache(config=model.config))
        cache = patch_model(model, bits=4, verify=True)
        got = _teacher_forced(model, ids, steps, cache)
        kinds = {i: type(lp).__name__ for i, lp in cache._pages.items()}
        unpatch_model(model)
        again = _teacher_forced(model, ids, steps, DynamicCache(config=model.config))
    assert kinds == {0: "_LayerFlat", 1: "_LayerPages", 2: "_LayerFlat", 3: "_LayerPages"}, kinds
    d0 = (got[:, 0] - ref[:, 0]).abs().max().item()
    print(f"[gemma4 patched vs unpatched] prefill logits max diff {d0:.3e}")
    assert torch.allclose(got[:, 0], ref[:, 0], atol=2e-2, rtol=2e-2)  # prefill: full precision
    cos = torch.nn.functional.cosine_similarity(got[0, 1:], ref[0, 1:], dim=-1)
    print(f"[gemma4 patched vs unpatched] decode logits cos per step {[round(c, 4) for c in cos.tolist()]}")
    assert cos.min() > 0.95 and cos.mean() > 0.975
    assert torch.equal(again, ref)


def test_flat_layer_decode_matches_dense(cuda):
    """A head dim without a paged kernel (64): the flat rows decode to the
    oracle's dequantised vectors and the decode attention equals float64
    softmax attention over them, per sequence length; with a window, only the
    last `window` positions and the first `sinks` are attended."""
    from fused_turboquant import TurboQuantMSE
    from fused_turboquant.hf import CompressedKVCache
    d, B, hkv, hq = 64, 2, 2, 8
    tq = TurboQuantMSE(d, bits=3, device=cuda)
    cache = CompressedKVCache(tq)
    cache.set_layer_quantizer(0, tq)
    g = torch.Generator().manual_seed(6)
    k = torch.randn(B, hkv, 21, d, generator=g).to(torch.bfloat16).to(cuda)
    v = torch.randn(B, hkv, 21, d, generator=g).to(torch.bfloat16).to(cuda)
    keep = torch.ones(B, 21, dtype=torch.bool)
    keep[1, :4] = False  # left padding of sequence 1
    cache.store_compressed_kv(k, v, 0, keep=keep.to(cuda))
    for _ in range(3):
        cache.store_compressed_kv(k[:, :, :1] * 0.5, v[:, :, :1] * 2, 0)
    assert cache.seq_lens(0) == [24, 20]
    q = torch.randn(B, hq, d, generator=g).to(torch.bfloat16).to(cuda)
    kd = cache.decode_keys(0).double().cpu().numpy()
    vd = cache.decode_values(0).double().cpu().numpy()
    for window, sinks in ((None, 0), (6, 2)):
        got = cache.decode_attention(q, 0, 0.125, sliding_window=window, sink_tokens=sinks).float().cpu().numpy()
        for b, L in enumerate((24, 20)):
            pos = np.arange(L)
            if window is not None:
                pos = pos[(pos >= L - window) | (pos < sinks)]
            for h in range(hq):
                s = kd[b, h // 4, pos] @ q[b, h].double().cpu().numpy() * 0.125
                p = np.exp(s - s.max())
                want = (p / p.sum()) @ vd[b, h // 4, pos]
                err = np.abs(got[b, h] - want).max()
                assert err <= 1e-2 + 2 ** -8 * np.abs(want).max(), (window, b, h, err)


def test_chunked_prefill_matches_one_pass(cuda):
    """chunked_prefill (reference hf/chunked_prefill.py:35-95): the next-token
    logits after a prompt prefilled in chunks of 7 follow a one-pass prefill
    of the same prompt to quantisation accuracy (each chunk attends over the
    compressed earlier chunks), and decode continues from the chunked cache."""
    from fused_turboquant.hf import patch_model, unpatch_model
    from fused_turboquant.hf.chunked_prefill import chunked_prefill
    model = _tiny_llama(cuda)
    ids = torch.randint(1, 320, (1, 40), generator=torch.Generator().manual_seed(8)).to(cuda)
    cache = patch_model(model, bits=4, verify=False)
    with torch.inference_mode():
        one = model(ids, past_key_values=cache, use_cache=True).logits[:, -1].float()
        cache.reset()
        chunked = chunked_prefill(model, ids, cache, chunk_size=7)[:, -1].float()
        assert cache.seq_lens(0) == [40]
        nxt = model(chunked.argmax(-1, keepdim=True), past_key_values=cache, use_cache=True).logits
    unpatch_model(model)
    cos = torch.nn.functional.cosine_similarity(one, chunked, dim=-1).min().item()
    print(f"[chunked prefill] last-token logits cos {cos:.4f}")
    assert cos > 0.98 and torch.isfinite(nxt).all()
