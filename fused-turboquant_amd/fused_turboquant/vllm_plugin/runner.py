"""A vLLM-style model runner for the ``TURBOQUANT`` backend: what vLLM's v1
engine does around ``FusedTurboQuantV1Impl`` on the decode path, without
vLLM.

vLLM is not installed on the machines this library is built and measured
on, so the pieces of vLLM that drive an attention backend are restated here
at the level the backend sees them (reference ``vllm_plugin/v1_backend.py``
``do_kv_cache_update`` ``:646-686`` and ``forward`` ``:755-836`` are called
exactly as vLLM's ``Attention`` layer calls them):

* ``BlockAllocator`` -- the KV-cache manager: one block table row per
  request, blocks taken from a seeded shuffle of the physical pages, so a
  sequence's pages are scattered the way they are after a server has run a
  while.
* ``StepMetadata`` -- the fields of vLLM's ``TurboQuantMetadata`` the
  backend reads (``num_actual_tokens``, ``is_prefill``, ``num_decodes``,
  ``num_decode_tokens``, ``seq_lens``, ``block_table``,
  ``query_start_loc``, ``max_query_len``, ``max_seq_len``, ``slot_mapping``;
  ``v1_backend.py:777-830``, ``1890-1919``).
* ``LlamaDecoder`` -- a Llama-architecture decoder in vLLM's flattened
  token layout ([num_tokens, hidden]): embedding, per layer RMSNorm, fused
  QKV projection, rotary embedding (in place on the QKV rows), the attention
  backend (store, then attention into a preallocated output), output
  projection with the residual add in the GEMM, RMSNorm, SwiGLU MLP; final
  norm and LM head on the sampled rows only.  Weights are drawn
  on the device from a seeded generator (no checkpoint is fetched).
* ``ModelRunner`` -- chunked prefill under a token budget
  (``max_num_batched_tokens``), greedy sampling, and decode steps captured
  once in a HIP graph and replayed (vLLM's CUDA-graph mode), with the step's
  positions, slots and sequence lengths computed on the device inside the
  graph.

The attention of each layer is either the ``TURBOQUANT`` Impl or
``DenseAttention``, a plain bf16 paged cache with torch SDPA, the baseline
the tests compare logits against.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Optional

import torch
import torch.nn.functional as F

from .v1_backend import FusedTurboQuantV1Backend, FusedTurboQuantV1Impl


@dataclass
class LlamaSpec:
    """Shape of a Llama-architecture decoder (defaults: Llama-3-8B)."""
    num_layers: int = 32
    hidden: int = 4096
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 14336
    vocab: int = 128256
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5
    max_positions: int = 8192


@dataclass
class StepMetadata:
    """The per-step attention metadata vLLM's metadata builder hands the
    backend (reference ``v1_backend.py:777-830``)."""
    num_actual_tokens: int
    is_prefill: bool
    num_decodes: int
    num_decode_tokens: int
    seq_lens: torch.Tensor         # int32 [B]
    block_table: torch.Tensor      # int32 [B, max_blocks]
    query_start_loc: torch.Tensor  # int32 [B + 1]
    max_query_len: int
    max_seq_len: int
    slot_mapping: torch.Tensor     # int64 [num_tokens]


class BlockAllocator:
    """Physical KV-cache pages handed to requests in a seeded random order
    (vLLM's block pool after churn), one block-table row per request."""

    def __init__(self, num_blocks: int, block_size: int, seed: int = 0):
        g = torch.Generator().manual_seed(seed)
        self.block_size = block_size
        self.free = torch.randperm(num_blocks, generator=g).tolist()

    def allocate(self, num_tokens: int) -> list[int]:
        n = (num_tokens + self.block_size - 1) // self.block_size
        if n > len(self.free):
            raise RuntimeError(f"KV cache out of blocks: need {n}, have {len(self.free)}")
        out, self.free = self.free[:n], self.free[n:]
        return out


class DenseAttention:
    """Baseline attention with the Impl's call surface: K and V kept in bf16
    pages ([num_blocks, block_size, Hkv, D] each, one layer's pair in
    ``kv_cache``), decode and prefill by torch SDPA over the gathered
    positions.  Used to compare logits, not for speed."""

    def __init__(self, num_heads: int, head_size: int, scale: float, num_kv_heads: int):
        self.num_heads, self.head_size, self.scale = num_heads, head_size, scale
        self.num_kv_heads = num_kv_heads

    @staticmethod
    def cache_shape(num_blocks, block_size, num_kv_heads, head_size):
        return (2, num_blocks, block_size, num_kv_heads, head_size)

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping):
        N = slot_mapping.shape[0]
        bs = kv_cache.shape[2]
        flat = kv_cache.view(2, -1, self.num_kv_heads, self.head_size)
        flat[0].index_copy_(0, slot_mapping[:N], key[:N].view(N, self.num_kv_heads, self.head_size))
        flat[1].index_copy_(0, slot_mapping[:N], value[:N].view(N, self.num_kv_heads, self.head_size))
        del bs

    def forward(self, layer, query, key, value, kv_cache, md, output):
        bs = kv_cache.shape[2]
        qsl = md.query_start_loc.tolist()
        sls = md.seq_lens.tolist()
        g = self.num_heads // self.num_kv_heads
        for i in range(len(sls)):
            a, b = qsl[i], qsl[i + 1]
            if b == a:
                continue
            L = sls[i]
            nblk = (L + bs - 1) // bs
            rows = md.block_table[i, :nblk].long()
            k = kv_cache[0, rows].reshape(-1, self.num_kv_heads, self.head_size)[:L]
            v = kv_cache[1, rows].reshape(-1, self.num_kv_heads, self.head_size)[:L]
            q = query[a:b].view(b - a, self.num_heads, self.head_size)
            qp = torch.arange(L - (b - a), L, device=q.device)
            mask = torch.arange(L, device=q.device)[None, :] <= qp[:, None]
            kk = k.transpose(0, 1).repeat_interleave(g, dim=0).float()
            vv = v.transpose(0, 1).repeat_interleave(g, dim=0).float()
            o = F.scaled_dot_product_attention(q.transpose(0, 1).float(), kk, vv, attn_mask=mask, scale=self.scale)
            output[a:b] = o.transpose(0, 1).reshape(b - a, -1).to(output.dtype)
        return output


class LlamaDecoder:
    """Llama-architecture decoder over vLLM's flattened tokens.  Weights are
    drawn on ``device`` with a seeded generator, in ``dtype``: a projection
    with fan-in n from N(0, 1/n) (unit-variance outputs for unit-variance
    inputs, so scores and activations keep a realistic spread), embeddings
    from N(0, 1), norm weights 1."""

    def __init__(self, spec: LlamaSpec, device, dtype=torch.bfloat16, seed: int = 0):
        self.spec, self.device, self.dtype = spec, torch.device(device), dtype
        g = torch.Generator(device=self.device).manual_seed(seed)
        s = spec
        q_out = s.num_heads * s.head_dim
        kv_out = s.num_kv_heads * s.head_dim

        def w(out, fan_in, std=None):
            t = torch.randn(out, fan_in, generator=g, device=self.device, dtype=torch.float32)
            return (t * (std if std is not None else fan_in ** -0.5)).to(dtype)

        self.embed = w(s.vocab, s.hidden, 1.0)
        self.layers = []
        for _ in range(s.num_layers):
            self.layers.append(SimpleNamespace(
                ln1=torch.ones(s.hidden, device=self.device, dtype=dtype),
                wqkv=w(q_out + 2 * kv_out, s.hidden),
                wo=w(s.hidden, q_out),
                ln2=torch.ones(s.hidden, device=self.device, dtype=dtype),
                wgu=w(2 * s.ffn, s.hidden),
                wd=w(s.hidden, s.ffn)))
        self.norm = torch.ones(s.hidden, device=self.device, dtype=dtype)
        self.lm_head = w(s.vocab, s.hidden)
        # rotary embedding as Llama's reference code states it: dims (2i, 2i + 1) form a
        # complex number turned by position * theta^(-2i / D) (the rotate-half form of other
        # implementations is the same map after a fixed permutation of the q / k weight rows)
        inv = 1.0 / (s.rope_theta ** (torch.arange(0, s.head_dim, 2, dtype=torch.float64) / s.head_dim))
        ang = torch.arange(s.max_positions, dtype=torch.float64)[:, None] * inv[None, :]
        self.freqs = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(self.device)

    def _rms(self, x, wgt):
        return F.rms_norm(x, (x.shape[-1],), wgt, self.spec.rms_eps)

    @staticmethod
    def _rope_(x, fc):
        """Rotary embedding in place on x [N, H, D] (fp32 arithmetic); fc:
        the complex rotations of the step's positions [N, 1, D / 2]."""
        xc = torch.view_as_complex(x.float().view(*x.shape[:-1], -1, 2))
        x.copy_(torch.view_as_real(xc * fc).view(x.shape))

    def forward(self, token_ids, positions, md: StepMetadata, attn, layer_objs, kv_caches, sample_rows,
                attn_hook=None):
        """Hidden states of all tokens through every layer, then the logits
        of the rows in ``sample_rows`` (int64 [S]) -> [S, vocab]."""
        s = self.spec
        N = token_ids.shape[0]
        q_out = s.num_heads * s.head_dim
        kv_out = s.num_kv_heads * s.head_dim
        fc = self.freqs[positions][:, None, :]  # once per step, shared by every layer
        x = self.embed[token_ids]
        for li, L in enumerate(self.layers):
            h = self._rms(x, L.ln1)
            qkv = F.linear(h, L.wqkv)
            self._rope_(qkv[:, :q_out + kv_out].view(N, s.num_heads + s.num_kv_heads, s.head_dim), fc)
            q2, k2, v = qkv[:, :q_out], qkv[:, q_out:q_out + kv_out], qkv[:, q_out + kv_out:]
            attn[li].do_kv_cache_update(layer_objs[li], k2, v, kv_caches[li], md.slot_mapping)
            o = torch.empty(N, q_out, dtype=x.dtype, device=x.device)
            attn[li].forward(layer_objs[li], q2, k2, v, kv_caches[li], md, output=o)
            if attn_hook is not None:
                attn_hook(li, q2, k2, v, o, md)
            x.addmm_(o, L.wo.t())  # residual add in the GEMM's epilogue
            h = self._rms(x, L.ln2)
            gu = F.linear(h, L.wgu)
            x.addmm_(F.silu(gu[:, :s.ffn]) * gu[:, s.ffn:], L.wd.t())
        hs = self._rms(x[sample_rows], self.norm)
        return F.linear(hs, self.lm_head)


class ModelRunner:
    """Prefill and greedy decode of a batch of requests through one
    attention backend per layer.

    ``backend``: ``"turboquant"`` (``FusedTurboQuantV1Impl`` with
    ``kv_cache_dtype``, the caches shaped by
    ``FusedTurboQuantV1Backend.get_kv_cache_shape``) or ``"dense"``
    (``DenseAttention``).  ``max_num_batched_tokens`` bounds the tokens of one
    prefill step (vLLM's chunked-prefill budget); a request's whole prompt
    goes into one step, several requests share a step while they fit.
    ``max_kv_splits``: the decode split-K factor fixed for graph capture
    (vLLM's ``tq_max_kv_splits_for_cuda_graph``); None sizes it for the
    longest context the run reaches."""

    def __init__(self, model: LlamaDecoder, max_batch: int, max_context: int, backend: str = "turboquant",
                 kv_cache_dtype: str = "turboquant_3bit_nc", block_size: int = 16,
                 max_num_batched_tokens: int = 16384, max_kv_splits: Optional[int] = None, seed: int = 0):
        s = model.spec
        self.model, self.backend, self.block_size = model, backend, block_size
        self.max_num_batched_tokens = max_num_batched_tokens
        dev = model.device
        self.device = dev
        blocks_per_seq = (max_context + block_size - 1) // block_size
        self.num_blocks = max_batch * blocks_per_seq + 8
        self.blocks_per_seq = blocks_per_seq
        scale = 1.0 / math.sqrt(s.head_dim)
        self.attn, self.layer_objs, self.kv_caches = [], [], []
        for _ in range(s.num_layers):
            if backend == "turboquant":
                impl = FusedTurboQuantV1Impl(s.num_heads, s.head_dim, scale, s.num_kv_heads,
                                             kv_cache_dtype=kv_cache_dtype)
                if max_kv_splits is not None:
                    impl.max_kv_splits = int(max_kv_splits)
                else:
                    from .. import v1 as V1
                    impl.max_kv_splits = max(1, int(V1.default_splits(max_batch, s.num_kv_heads, max_context)))
                shape = FusedTurboQuantV1Backend.get_kv_cache_shape(self.num_blocks, block_size, s.num_kv_heads,
                                                                    s.head_dim, kv_cache_dtype)
                cache = torch.zeros(shape, dtype=torch.uint8, device=dev)
            elif backend == "dense":
                impl = DenseAttention(s.num_heads, s.head_dim, scale, s.num_kv_heads)
                cache = torch.zeros(DenseAttention.cache_shape(self.num_blocks, block_size, s.num_kv_heads,
                                                               s.head_dim), dtype=model.dtype, device=dev)
            else:
                raise ValueError(f"backend must be 'turboquant' or 'dense', got {backend!r}")
            self.attn.append(impl)
            self.layer_objs.append(SimpleNamespace())
            self.kv_caches.append(cache)
        self._seed = seed
        self.alloc = BlockAllocator(self.num_blocks, block_size, seed)
        self.max_batch = max_batch
        self.graph = None
        # attn_hook(layer_index, query, key, value, output, metadata): called after each layer's
        # attention in eager steps (tests); keep_logits: eager steps append their logits to .logits
        self.attn_hook = None
        self.keep_logits = False
        self.logits: list[torch.Tensor] = []

    def reset(self):
        """Return every page to the pool (a new batch of requests; the cache
        bytes are left as they are, every slot is written before it is read)."""
        self.alloc = BlockAllocator(self.num_blocks, self.block_size, self._seed)
        self.graph = None

    # -- prefill -------------------------------------------------------------
    def prefill(self, prompts: list[torch.Tensor]) -> tuple[torch.Tensor, torch.Tensor]:
        """Fresh prefill of every prompt (int64 token ids on the device), in
        steps of at most ``max_num_batched_tokens`` tokens.  Returns the block
        table (int32 [B, blocks_per_seq]) and the first sampled token of each
        request (int64 [B])."""
        dev, bs = self.device, self.block_size
        B = len(prompts)
        if B > self.max_batch:
            raise ValueError(f"{B} requests > max_batch {self.max_batch}")
        bt = torch.zeros(B, self.blocks_per_seq, dtype=torch.int32)
        for i, p in enumerate(prompts):
            blocks = self.alloc.allocate(self.blocks_per_seq * bs)
            bt[i] = torch.tensor(blocks, dtype=torch.int32)
        bt = bt.to(dev)
        first = torch.empty(B, dtype=torch.int64, device=dev)
        i = 0
        while i < B:
            j, tok = i, 0
            while j < B and (j == i or tok + prompts[j].numel() <= self.max_num_batched_tokens):
                tok += prompts[j].numel()
                j += 1
            lens = [int(prompts[r].numel()) for r in range(i, j)]
            ids = torch.cat(prompts[i:j])
            pos = torch.cat([torch.arange(n, device=dev) for n in lens])
            rows = torch.cat([torch.full((n,), r, device=dev, dtype=torch.int64) for r, n in zip(range(i, j), lens)])
            slots = bt[rows, pos // bs].long() * bs + pos % bs
            qsl = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=dev)
            md = StepMetadata(num_actual_tokens=tok, is_prefill=True, num_decodes=0, num_decode_tokens=0,
                              seq_lens=torch.tensor(lens, dtype=torch.int32, device=dev), block_table=bt[i:j],
                              query_start_loc=qsl, max_query_len=max(lens), max_seq_len=max(lens),
                              slot_mapping=slots)
            last = (qsl[1:] - 1).long()
            logits = self.model.forward(ids, pos, md, self.attn, self.layer_objs, self.kv_caches, last,
                                        attn_hook=self.attn_hook)
            if self.keep_logits:
                self.logits.append(logits)
            first[i:j] = logits.argmax(dim=-1)
            i = j
        return bt, first

    # -- decode --------------------------------------------------------------
    def _decode_body(self):
        st = self._st
        bs = self.block_size
        pos = st.pos
        seq_lens = (pos + 1).to(torch.int32)
        slots = st.bt.gather(1, (pos // bs)[:, None]).squeeze(1).long() * bs + pos % bs
        md = StepMetadata(num_actual_tokens=st.B, is_prefill=False, num_decodes=st.B, num_decode_tokens=st.B,
                          seq_lens=seq_lens, block_table=st.bt, query_start_loc=st.qsl, max_query_len=1,
                          max_seq_len=st.max_seq_len, slot_mapping=slots)
        capturing = self.device.type == "cuda" and torch.cuda.is_current_stream_capturing()
        logits = self.model.forward(st.tok, pos, md, self.attn, self.layer_objs, self.kv_caches, st.rows,
                                    attn_hook=None if capturing else self.attn_hook)
        if self.keep_logits and not capturing:
            self.logits.append(logits)
        nxt = logits.argmax(dim=-1)
        st.out.index_copy_(0, st.step, nxt[None])
        st.tok.copy_(nxt)
        st.pos.add_(1)
        st.step.add_(1)

    def start_decode(self, block_table: torch.Tensor, first_tokens: torch.Tensor, prompt_lens: list[int],
                     max_steps: int, use_graph: bool = True):
        """Device state of a decode run: the last sampled tokens, their
        positions, the output buffer [max_steps, B]; with ``use_graph`` one
        decode step is captured in a HIP graph (after a warm-up step on a side
        stream that allocates every per-layer buffer, undone afterwards)."""
        dev = self.device
        B = first_tokens.shape[0]
        self._st = SimpleNamespace(
            B=B, bt=block_table, tok=first_tokens.clone(), rows=torch.arange(B, device=dev),
            pos=torch.tensor(prompt_lens, dtype=torch.int64, device=dev),
            qsl=torch.arange(B + 1, dtype=torch.int32, device=dev),
            out=torch.zeros(max_steps, B, dtype=torch.int64, device=dev),
            step=torch.zeros(1, dtype=torch.int64, device=dev),
            max_seq_len=max(prompt_lens) + max_steps)
        self.graph = None
        if use_graph:
            st = self._st
            saved = (st.tok.clone(), st.pos.clone(), st.out.clone(), st.step.clone())
            side = torch.cuda.Stream(device=dev)
            side.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(side):
                self._decode_body()  # allocates the per-layer scratch outside the capture
            torch.cuda.current_stream(dev).wait_stream(side)
            torch.cuda.synchronize(dev)
            st.tok.copy_(saved[0])
            st.pos.copy_(saved[1])
            st.out.copy_(saved[2])
            st.step.copy_(saved[3])
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._decode_body()
            # the capture recorded the step without running it: state is still the start
            self.graph = g

    def decode_step(self, force: Optional[torch.Tensor] = None):
        """One decode step of every request; ``force`` (int64 [B]) replaces
        the sampled tokens as the next step's input (teacher forcing, to
        compare two backends on one token sequence)."""
        if self.graph is not None:
            self.graph.replay()
        else:
            self._decode_body()
        if force is not None:
            self._st.tok.copy_(force)

    def decoded_tokens(self) -> torch.Tensor:
        return self._st.out

    def generate(self, prompts: list[torch.Tensor], max_new_tokens: int, use_graph: bool = True) -> torch.Tensor:
        """Greedy generation: [B, max_new_tokens] int64 (the first token from
        the prefill logits, the rest from max_new_tokens - 1 decode steps)."""
        bt, first = self.prefill(prompts)
        steps = max_new_tokens - 1
        self.start_decode(bt, first, [int(p.numel()) for p in prompts], max(steps, 1), use_graph=use_graph)
        for _ in range(steps):
            self.decode_step()
        return torch.cat([first[:, None], self._st.out[:steps].t()], dim=1)
