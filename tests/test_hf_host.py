"""HF integration host logic on the CPU: page reader vs the oracle's, argument
checks, compatibility report, quantizer routing (no kernel calls)."""
import numpy as np
import pytest
import torch

from oracle import tq_oracle as O


@pytest.mark.parametrize("d,bk,bv", [(128, 3, 3), (128, 4, 2), (256, 2, 4)])
def test_paged_read_matches_oracle_page_reader(d, bk, bv):
    from fused_turboquant import paged as P
    rng = np.random.default_rng(d + bk * 7 + bv)
    shape = P.cache_shape(5, 32, 2, d, bk, bv)
    cache = rng.integers(0, 256, size=shape, dtype=np.uint8)
    # keep the norm bytes finite fp16 (exponent < 31) so views compare cleanly
    sub = shape[-1]
    cache[..., sub - 64 + 1::2] &= 0x7B
    blocks = torch.tensor([3, 0, 4])
    kp, kn, vp, vn = P.paged_read(torch.from_numpy(cache), blocks, d, bk, bv)
    kc, vc, kn_o, vn_o = O.paged_unpack(cache, d, bk, bv)
    sel = blocks.numpy()
    assert np.array_equal(O.unpack(kp.numpy(), bk, d), kc[sel])
    assert np.array_equal(O.unpack(vp.numpy(), bv, d), vc[sel])
    assert np.array_equal(kn.numpy(), kn_o[sel])
    assert np.array_equal(vn.numpy(), vn_o[sel])


def test_patch_model_rejects_bad_bits():
    from fused_turboquant.hf import patch_model

    class _Dummy:
        pass

    with pytest.raises(ValueError, match="v_bits"):
        patch_model(_Dummy(), bits=4, v_bits=5)
    with pytest.raises(ValueError, match="bits"):
        patch_model(_Dummy(), bits=5)
    with pytest.raises(NotImplementedError):
        patch_model(_Dummy(), quantizer_kind="planar")
    with pytest.raises(ValueError, match="boundary_protect"):
        patch_model(_Dummy(), boundary_protect=-1)


def _tiny_llama(head_dim=128, layers=2, heads=4, kv_heads=2):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(hidden_size=heads * head_dim, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=head_dim,
                      vocab_size=320, max_position_embeddings=512)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg)


def test_check_model_compatibility():
    from fused_turboquant.hf import check_model_compatibility
    r = check_model_compatibility(_tiny_llama())
    assert r["compatible"] and r["eligible_layers"] == 2 and r["head_dim"] == 128
    assert r["n_q_heads"] == 4 and r["n_kv_heads"] == 2 and r["known_compatible"]
    r64 = check_model_compatibility(_tiny_llama(head_dim=64))  # flat rows + torch attention
    assert r64["compatible"] and r64["head_dims"] == [64] and r64["paged_head_dims"] == []
    r96 = check_model_compatibility(_tiny_llama(head_dim=96))
    assert not r96["compatible"] and any("head_dim" in i for i in r96["issues"])


def test_quantizer_routing():
    from fused_turboquant import TurboQuantMSE
    from fused_turboquant.hf import CompressedKVCache
    k_tq = TurboQuantMSE(128, bits=4)
    v_tq = TurboQuantMSE(128, bits=3)
    cache = CompressedKVCache(k_tq)
    cache.set_layer_quantizer(0, k_tq)
    assert cache.get_layer_quantizer_v(0) is k_tq  # V falls back to K
    cache.set_layer_quantizer_v(0, v_tq)
    assert cache.get_layer_quantizer(0) is k_tq and cache.get_layer_quantizer_v(0) is v_tq
    assert cache.get_layer_quantizer(7) is k_tq  # unregistered layer -> default


class _ResettableCache:
    """A transformers DynamicCache with the ``reset()`` the smoke test calls."""

    def __new__(cls):
        from transformers import DynamicCache

        class _C(DynamicCache):
            def reset(self):
                self.__init__()
        return _C()


def _swap_attention(model, make):
    """Replace every self-attention forward by make(original); returns the originals."""
    originals = {}
    for name, module in model.named_modules():
        if name.endswith("self_attn"):
            originals[name] = module.forward
            module.forward = make(module.forward)
    return originals


def test_smoke_test_compares_against_unpatched_logits():
    """The verify step runs prompt + decode through the patched forwards and
    the same tokens through the originals, and passes on identical paths
    (cosine 1), leaving the patched forwards installed."""
    from fused_turboquant.hf import fused_cache as FC
    model = _tiny_llama().eval()
    originals = _swap_attention(model, lambda f: (lambda *a, **k: f(*a, **k)))
    patched = {n: m.forward for n, m in model.named_modules() if n in originals}
    cos = FC._smoke_test(model, _ResettableCache(), originals, model.config)
    assert cos == pytest.approx(1.0, abs=1e-5)
    assert all(m.forward is patched[n] for n, m in model.named_modules() if n in originals)


def test_smoke_test_rejects_a_wrong_attention_path():
    """A patched attention that returns the wrong output (negated here, on the
    CPU) drives the logit cosine below 0.8 and fails the verify step; the
    patched forwards are still the installed ones afterwards."""
    from fused_turboquant.hf import fused_cache as FC
    model = _tiny_llama().eval()

    def wrong(f):
        def fwd(*a, **k):
            out = f(*a, **k)
            return (-4.0 * out[0],) + tuple(out[1:])
        return fwd
    originals = _swap_attention(model, wrong)
    patched = {n: m.forward for n, m in model.named_modules() if n in originals}
    with pytest.raises(RuntimeError, match="cosine similarity"):
        FC._smoke_test(model, _ResettableCache(), originals, model.config)
    assert all(m.forward is patched[n] for n, m in model.named_modules() if n in originals)


def _tiny_gemma4(shared=0):
    from transformers import Gemma4TextConfig
    from transformers.models.gemma4.modeling_gemma4 import Gemma4ForCausalLM
    cfg = Gemma4TextConfig(vocab_size=320, hidden_size=256, intermediate_size=512, num_hidden_layers=4,
                           num_attention_heads=4, num_key_value_heads=2, head_dim=64, global_head_dim=128,
                           sliding_window=8,
                           layer_types=["sliding_attention", "full_attention", "sliding_attention", "full_attention"],
                           attention_k_eq_v=True, num_global_key_value_heads=1, vocab_size_per_layer_input=320,
                           hidden_size_per_layer_input=16, max_position_embeddings=512, num_kv_shared_layers=shared)
    torch.manual_seed(0)
    return Gemma4ForCausalLM(cfg)


def test_gemma4_compatibility_report():
    """Gemma 4: per-layer head dims (64 sliding, 128 full), K = V full layers,
    sliding windows, scaling 1.0 -- reported compatible; KV-shared layers are
    reported and refused by patch_model (reference hf/fused_cache.py:421-426)."""
    from fused_turboquant.hf import check_model_compatibility, patch_model
    from fused_turboquant.hf import fused_cache as FC
    m = _tiny_gemma4()
    r = check_model_compatibility(m)
    assert r["compatible"], r["issues"]
    assert r["head_dims"] == [64, 128] and r["paged_head_dims"] == [128] and r["k_eq_v_layers"] == 2
    attn = [mod for n, mod in m.named_modules() if n.endswith("self_attn")]
    assert [FC._resolve_layer_head_dim(a, m.config) for a in attn] == [64, 128, 64, 128]
    assert [FC._layer_sliding_window(a, m.config) for a in attn] == [8, None, 8, None]
    assert [FC._module_k_eq_v(a) for a in attn] == [False, True, False, True]
    s = _tiny_gemma4(shared=2)
    r = check_model_compatibility(s)
    assert not r["compatible"] and r["kv_shared_layers"] == 2
    with pytest.raises(ValueError, match="KV-shared"):
        patch_model(s, bits=4)


def test_keep_and_window_masks():
    """Padding detection reads each token from the last query row whose
    window holds it; the continuation mask limits rows to their window."""
    from fused_turboquant.hf import fused_cache as FC
    q, W = 6, 3
    i = torch.arange(q)
    vis = (i[None, :] <= i[:, None]) & (i[None, :] > i[:, None] - W)   # sliding causal
    vis = vis[None, None].repeat(2, 1, 1, 1)
    vis[1, :, :, :2] = False                                          # sequence 1: two padding tokens
    keep = FC._keep_from_mask(vis, q, W)
    assert keep.tolist() == [[True] * 6, [False, False, True, True, True, True]]
    assert FC._keep_from_mask(vis[:1], q, W) is None
    m = FC._continuation_mask([5, 2], 5, 3, None, None, True, "cpu", window=4)[:, 0]
    # sequence 0: rows at positions 5, 6, 7 see positions > p - 4 of its 5 past + itself causally
    assert m[0, 0].tolist() == [False, False, True, True, True, True, False, False]
    assert m[0, 2].tolist() == [False, False, False, False, True, True, True, True]
    # sequence 1: 2 past positions (2..4 of the decoded past are not its own)
    assert m[1, 0].tolist() == [True, True, False, False, False, True, False, False]
