"""Chunked prefill with incremental KV compression (reference
``hf/chunked_prefill.py:35-177``).

A long prompt goes through the patched model in chunks of ``chunk_size``
tokens; each chunk's K / V are compressed into the cache as the chunk runs,
so the full-precision K / V of at most one chunk exist at a time.  A chunk
after the first attends over the decoded cache of the earlier chunks plus
itself, causally (the patched forward's multi-token path).
"""
from __future__ import annotations

import logging

import torch

from .fused_cache import CompressedKVCache, patch_model, unpatch_model

logger = logging.getLogger(__name__)


def chunked_prefill(model, input_ids: torch.Tensor, cache: CompressedKVCache, chunk_size: int = 2048,
                    attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Run ``input_ids`` [B, S] through the patched ``model`` in chunks of
    ``chunk_size`` tokens, filling ``cache``; returns the last chunk's logits.
    ``attention_mask`` [B, S] (1 = token, 0 = left padding) is passed on with
    the positions of each chunk."""
    if chunk_size < 1:
        raise ValueError("chunk_size must be >= 1")
    S = input_ids.shape[1]
    if attention_mask is None:
        attention_mask = torch.ones_like(input_ids)
    position_ids = (attention_mask.long().cumsum(-1) - 1).clamp(min=0)
    n_chunks = (S + chunk_size - 1) // chunk_size
    if n_chunks > 1:
        logger.info("Chunked prefill: %d tokens in %d chunks of %d", S, n_chunks, chunk_size)
    logits = None
    for i in range(n_chunks):
        a, b = i * chunk_size, min((i + 1) * chunk_size, S)
        with torch.inference_mode():
            out = model(input_ids[:, a:b], attention_mask=attention_mask[:, :b], position_ids=position_ids[:, a:b],
                        past_key_values=cache, use_cache=True)
        logits = out.logits
    return logits


def chunked_generate(model, tokenizer, prompt: str, bits: int = 4, chunk_size: int = 2048,
                     max_new_tokens: int = 200, do_sample: bool = False, compress_v: bool | str = True,
                     verify: bool = False) -> str:
    """Patch ``model``, prefill ``prompt`` in chunks, generate up to
    ``max_new_tokens`` tokens (greedy unless ``do_sample``; stops at the
    tokenizer's EOS), unpatch, and return the generated text."""
    cache = patch_model(model, bits=bits, compress_v=compress_v, verify=verify)
    try:
        ids = tokenizer(prompt, return_tensors="pt").to(model.device)["input_ids"]
        logits = chunked_prefill(model, ids, cache, chunk_size=chunk_size)

        def pick(lg):
            if do_sample:
                return torch.multinomial(torch.softmax(lg.float(), dim=-1), 1)
            return lg.argmax(dim=-1, keepdim=True)
        tok = pick(logits[:, -1])
        gen = [tok]
        eos = getattr(tokenizer, "eos_token_id", None)
        with torch.inference_mode():
            for _ in range(max_new_tokens - 1):
                if eos is not None and int(tok.item()) == eos:
                    break
                tok = pick(model(tok, past_key_values=cache, use_cache=True).logits[:, -1])
                gen.append(tok)
        return tokenizer.decode(torch.cat(gen, dim=1)[0], skip_special_tokens=True)
    finally:
        unpatch_model(model)
