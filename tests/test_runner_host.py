"""The vLLM-style model runner's own bookkeeping, on the CPU with the dense
bf16-cache baseline attention (no GPU kernel involved): block tables, slot
mapping, positions, chunked prefill and decode steps must give the logits a
from-scratch prefill of the same tokens gives."""
import torch

from conftest import ROOT  # noqa: F401  (puts the package on sys.path)


def _model():
    from fused_turboquant.vllm_plugin.runner import LlamaDecoder, LlamaSpec
    spec = LlamaSpec(num_layers=2, hidden=256, num_heads=8, num_kv_heads=2, head_dim=64, ffn=384, vocab=257,
                     max_positions=128)
    return LlamaDecoder(spec, "cpu", dtype=torch.float32, seed=3)


def test_decode_steps_equal_full_prefill():
    from fused_turboquant.vllm_plugin.runner import ModelRunner
    m = _model()
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, 257, (n,), generator=g) for n in (21, 9, 30)]
    run = ModelRunner(m, max_batch=3, max_context=48, backend="dense", max_num_batched_tokens=32, block_size=16)
    run.keep_logits = True
    toks = run.generate(prompts, 6, use_graph=False)
    n_prefill = len(run.logits) - 5
    assert n_prefill == 2  # 21 + 9 tokens in the first step (budget 32), 30 in the second
    dec = run.logits[n_prefill:]
    for s in (0, 2, 4):
        # the logits of decode step s (input token toks[:, s]) = a fresh prefill of prompt + toks[:, :s + 1]
        ext = [torch.cat([p, toks[i, :s + 1]]) for i, p in enumerate(prompts)]
        ref = ModelRunner(m, max_batch=3, max_context=48, backend="dense", max_num_batched_tokens=64, block_size=16,
                          seed=9)
        ref.keep_logits = True
        ref.prefill(ext)
        want = torch.cat(ref.logits)
        assert torch.allclose(dec[s], want, atol=1e-4, rtol=1e-4), s


def test_block_allocator_hands_out_each_page_once():
    from fused_turboquant.vllm_plugin.runner import BlockAllocator
    a = BlockAllocator(10, 16, seed=4)
    got = a.allocate(33) + a.allocate(16) + a.allocate(1)
    assert len(got) == 5 and len(set(got)) == 5 and all(0 <= b < 10 for b in got)
    import pytest
    with pytest.raises(RuntimeError):
        a.allocate(16 * 6)
