"""End-to-end generation on the Qwen3 decoder architecture over the gfx950 attention path.

A whole-model throughput harness around the drop-in layers:

* ``Qwen3Config`` / ``Qwen3ForCausalLM`` - the decoder of
  src/nano_inference/models/qwen3.py:19-150 (embedding, per block
  RMSNorm -> PagedCausalSelfAttention -> residual -> RMSNorm -> SwiGLU MLP ->
  residual, final RMSNorm, optionally tied LM head), with this package's
  ``PagedCausalSelfAttention`` as its attention layer and random-initialised
  weights (no checkpoint is loaded).
* ``KVPool`` - the reference allocator's cache layout, one
  ``[layers, blocks, kv_heads, block_size, head_dim]`` tensor each for K and V
  (src/nano_inference/kv_cache/allocator.py:35-39), with a free list of blocks.
* ``Generator`` - prefill first: waiting prompts enter in prefill steps of up to
  ``max_prefill_batch`` sequences (padded (B, S_max) batches with a prefix
  attention mask, as the reference batches prefill), then every running sequence
  decodes one token per step, the decode step captured once in a HIP graph.
* ``MixedGenerator`` - continuous batching with chunked prefill: each step packs
  one token of every decoding sequence and prefill chunks of the others into one
  row of tokens (``ChunkedScheduler`` plans it; ``PackedAttentionMetadata``
  routes decode rows to the decode kernel and chunk rows to the chunked-prefill
  kernel); step metadata is one descriptor expanded on the device, sampled tokens
  stay on the device, and the all-decode tail replays one HIP graph.  The
  reference's scheduler runs prefill and decode in separate batches and gives
  decode priority (src/nano_inference/scheduler/scheduler.py:125-230).
* Either generator can keep the KV pool in the fp8 format (``fp8_cache``).
* Sampling is greedy on each sequence's last valid position (the reference takes
  position S_step - 1 of the padded batch for every row,
  src/nano_inference/inferencer/torch_inferencer.py:242-251, which for shorter
  prompts of a padded prefill batch is a padding position).

Throughput is the reference's metric: (prompt + generated tokens) / elapsed
(src/nano_inference/scheduler/scheduler.py:352-364).
"""
from __future__ import annotations

import math
import time
from collections import deque
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .attention import PagedCausalSelfAttention
from .context import AttentionMetadata, PackedAttentionMetadata
from .layers import RMSNorm


@dataclass
class Qwen3Config:
    """Qwen3-0.6B architecture (the public config's sizes)."""

    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    num_layers: int = 28
    rms_norm_eps: float = 1e-6
    rope_base: float = 1e6
    use_qk_norm: bool = True
    tie_word_embeddings: bool = True


class SwiGLUMLP(nn.Module):
    """down(silu(gate(x)) * up(x)), as src/nano_inference/layers/mlp.py."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class Qwen3DecoderBlock(nn.Module):
    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        self.input_norm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)
        self.self_attn = PagedCausalSelfAttention(
            cfg.hidden_size, cfg.num_heads, num_kv_heads=cfg.num_kv_heads,
            head_dim=cfg.head_dim, use_qk_norm=cfg.use_qk_norm, rope_base=cfg.rope_base)
        self.post_attention_norm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)
        self.mlp = SwiGLUMLP(cfg.hidden_size, cfg.intermediate_size)

    def forward(self, x, position_ids, attention_mask, metadata):
        x = x + self.self_attn(self.input_norm(x), position_ids=position_ids,
                               attention_mask=attention_mask, metadata=metadata)
        return x + self.mlp(self.post_attention_norm(x))


class Qwen3ForCausalLM(nn.Module):
    """Decoder + LM head; ``forward`` returns logits at the selected positions only."""

    def __init__(self, cfg: Qwen3Config):
        super().__init__()
        self.config = cfg
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(Qwen3DecoderBlock(cfg) for _ in range(cfg.num_layers))
        for i, layer in enumerate(self.layers):
            layer.self_attn.layer_idx = i
        self.norm = RMSNorm(cfg.hidden_size, eps=cfg.rms_norm_eps)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        if cfg.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight

    @torch.no_grad()
    def init_random(self, seed: int, std: float = 0.02) -> "Qwen3ForCausalLM":
        """Seeded N(0, std) weights for every matrix, ones for the norms."""
        g = torch.Generator(device="cpu").manual_seed(seed)
        for name, prm in self.named_parameters():
            if name.endswith("norm.weight"):
                prm.fill_(1.0)
            else:
                prm.copy_(torch.randn(prm.shape, generator=g) * std)
        return self

    def forward(self, input_ids, position_ids, attention_mask, metadata, select):
        """input_ids (B, S); ``select`` (B,) index of the position whose logits to return."""
        x = self.embed_tokens(input_ids)
        for layer in self.layers:
            x = layer(x, position_ids, attention_mask, metadata)
        last = x[torch.arange(x.shape[0], device=x.device), select]
        return self.lm_head(self.norm(last))


    def forward_packed(self, input_ids, position_ids, metadata, rows):
        """A packed step: input_ids / position_ids (T,), logits at packed ``rows``."""
        x = self.embed_tokens(input_ids).unsqueeze(0)
        pos = position_ids.unsqueeze(0)
        for layer in self.layers:
            x = layer(x, pos, None, metadata)
        return self.lm_head(self.norm(x[0, rows]))


class KVPool:
    """Paged K/V caches of all layers plus a free list of their blocks.  With
    ``fp8`` the caches hold e4m3 codes (uint8) with one fp32 scale per
    (block, KV head, slot) row in ``k_scale`` / ``v_scale``.  The layout is checked
    against every kernel the pool feeds when it is built (ops.check_pool_shape)."""

    def __init__(self, cfg: Qwen3Config, num_blocks: int, block_size: int, dtype, device,
                 fp8: bool = False):
        ops.check_pool_shape(cfg.head_dim, block_size, cfg.num_heads, cfg.num_kv_heads,
                             dtype, fp8)
        shape = (cfg.num_layers, num_blocks, cfg.num_kv_heads, block_size, cfg.head_dim)
        cdt = torch.uint8 if fp8 else dtype
        self.k_cache = torch.zeros(shape, dtype=cdt, device=device)
        self.v_cache = torch.zeros(shape, dtype=cdt, device=device)
        self.k_scale = self.v_scale = None
        if fp8:
            self.k_scale = torch.zeros(shape[:4], dtype=torch.float32, device=device)
            self.v_scale = torch.zeros(shape[:4], dtype=torch.float32, device=device)
        self.block_size = block_size
        self.free: deque = deque(range(num_blocks))

    def allocate(self, tokens: int) -> List[int]:
        n = math.ceil(tokens / self.block_size)
        if n > len(self.free):
            raise RuntimeError(f"KV pool exhausted: {n} blocks wanted, {len(self.free)} free")
        return [self.free.popleft() for _ in range(n)]

    def release(self, blocks: List[int]) -> None:
        self.free.extend(blocks)


def _graph_workspace(model, pool: KVPool, block_tables: torch.Tensor) -> torch.Tensor:
    """A decode workspace owned by the generator for the decode steps it captures in a HIP
    graph (batch and table width fixed), released with the graph when the run ends."""
    cfg = model.config
    qdt = torch.bfloat16 if pool.k_scale is not None else pool.k_cache.dtype
    n = ops.decode_workspace_bytes(block_tables.shape[0], cfg.num_heads, cfg.num_kv_heads,
                                   block_tables.shape[1], pool.block_size, cfg.head_dim, qdt)
    return torch.empty(max(n, 1), dtype=torch.uint8, device=block_tables.device)


@dataclass
class _Seq:
    prompt: List[int]
    blocks: List[int]
    generated: List[int] = field(default_factory=list)


@dataclass
class GenerationStats:
    prompt_tokens: int = 0
    generated_tokens: int = 0
    prefill_steps: int = 0
    decode_steps: int = 0
    prefill_s: float = 0.0
    decode_s: float = 0.0
    total_s: float = 0.0

    @property
    def tokens_per_s(self) -> float:
        return (self.prompt_tokens + self.generated_tokens) / self.total_s

    @property
    def decode_tokens_per_s(self) -> float:
        return self.generated_tokens / self.decode_s if self.decode_s > 0 else 0.0


class Generator:
    """Greedy generation of fixed-length continuations (no EOS) for a set of prompts."""

    def __init__(self, model: Qwen3ForCausalLM, pool: KVPool, max_new_tokens: int,
                 max_prefill_batch: int = 8, max_blocks_per_seq: Optional[int] = None,
                 use_graph: bool = False):
        self.model = model
        self.pool = pool
        self.max_new = max_new_tokens
        self.max_prefill_batch = max_prefill_batch
        self.max_blocks = max_blocks_per_seq
        self.use_graph = use_graph
        self.replay_hook = None  # called after every graph replay (tests interleave work)
        self.device = pool.k_cache.device

    # ---- metadata ---------------------------------------------------------------------
    def _tables(self, seqs: List[_Seq]) -> torch.Tensor:
        width = self.max_blocks or max(len(s.blocks) for s in seqs)
        bt = torch.zeros((len(seqs), width), dtype=torch.int32)
        for i, s in enumerate(seqs):
            bt[i, :len(s.blocks)] = torch.tensor(s.blocks, dtype=torch.int32)
        return bt

    def _prefill_inputs(self, seqs: List[_Seq]):
        bs = self.pool.block_size
        lens = torch.tensor([len(s.prompt) for s in seqs], dtype=torch.int64)
        b, smax = len(seqs), int(lens.max())
        ids = torch.zeros((b, smax), dtype=torch.int64)
        for i, s in enumerate(seqs):
            ids[i, :len(s.prompt)] = torch.tensor(s.prompt, dtype=torch.int64)
        pos = torch.arange(smax, dtype=torch.int64).unsqueeze(0).expand(b, smax)
        valid = pos < lens.unsqueeze(1)
        bt = self._tables(seqs)
        blk = torch.gather(bt.to(torch.int64), 1, (pos // bs).clamp(max=bt.shape[1] - 1))
        slots = torch.where(valid, blk * bs + pos % bs, torch.full_like(pos, -1))
        dev = self.device
        md = AttentionMetadata(context_lens=lens.to(dev), kv_block_tables=bt.to(dev),
                               slot_mapping=slots.to(dev), k_cache=self.pool.k_cache,
                               v_cache=self.pool.v_cache, k_scale=self.pool.k_scale,
                               v_scale=self.pool.v_scale, is_prefill=True)
        return (ids.to(dev), pos.contiguous().to(dev), valid.to(dev), md,
                (lens - 1).to(dev))

    # ---- steps ------------------------------------------------------------------------
    @torch.no_grad()
    def run(self, prompts: List[List[int]]) -> GenerationStats:
        st = GenerationStats(prompt_tokens=sum(len(p) for p in prompts))
        waiting = deque(prompts)
        running: List[_Seq] = []
        dev = self.device
        sync = torch.cuda.synchronize if dev.type == "cuda" else (lambda: None)
        sync()
        t0 = time.perf_counter()
        # Prefill priority: all waiting prompts enter before decoding starts.
        while waiting:
            batch = [_Seq(p, self.pool.allocate(len(p) + self.max_new))
                     for p in (waiting.popleft() for _ in range(min(self.max_prefill_batch,
                                                                   len(waiting))))]
            ids, pos, mask, md, last = self._prefill_inputs(batch)
            logits = self.model(ids, pos, mask, md, last)
            nxt = torch.argmax(logits, dim=-1)
            for i, s in enumerate(batch):
                s.generated.append(nxt[i])
            running.extend(batch)
            st.prefill_steps += 1
        sync()
        t1 = time.perf_counter()
        # Decode: every sequence is the same step further along, so a step's tensors
        # follow on the device from a step counter; the step (metadata, model, argmax,
        # history write, counter update) has fixed shapes and addresses, so it can be
        # captured once into a HIP graph and replayed.
        if running and self.max_new > 1:
            b = len(running)
            self._bt = self._tables(running).to(dev)
            self._lens = torch.tensor([len(s.prompt) for s in running], dtype=torch.int64,
                                      device=dev)
            self._rows = torch.arange(b, device=dev)
            self._zero = torch.zeros(b, dtype=torch.int64, device=dev)
            self._hist = torch.zeros((b, self.max_new), dtype=torch.int64, device=dev)
            self._hist[:, 0] = torch.stack([s.generated[0] for s in running]).to(torch.int64)
            self._step = torch.ones(1, dtype=torch.int64, device=dev)  # index being produced
            self._ws = _graph_workspace(self.model, self.pool, self._bt)
            self._decode_step()  # eager first step (also warms up the libraries)
            st.decode_steps += 1
            if self.use_graph and self.max_new > 2:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    self._decode_step()
                for _ in range(2, self.max_new):
                    graph.replay()
                    st.decode_steps += 1
                    if self.replay_hook is not None:
                        self.replay_hook()
            else:
                for _ in range(2, self.max_new):
                    self._decode_step()
                    st.decode_steps += 1
            gen = self._hist.cpu()
            for i, s in enumerate(running):
                s.generated = gen[i].tolist()
        sync()
        t2 = time.perf_counter()
        for s in running:
            self.pool.release(s.blocks)
        st.generated_tokens = len(running) * self.max_new
        st.prefill_s, st.decode_s, st.total_s = t1 - t0, t2 - t1, t2 - t0
        self.outputs = [s.generated for s in running]
        return st


    def _decode_positions(self):
        """Position, slot and context length of the token every sequence feeds at the
        current step (the step produces token ``step``, feeding token ``step - 1``)."""
        bs = self.pool.block_size
        p = self._lens + self._step - 1
        slot = self._bt[self._rows, p // bs].to(torch.int64) * bs + p % bs
        return p, slot, p + 1

    def _decode_step(self) -> None:
        """Feed token ``step - 1`` of every sequence and write token ``step``."""
        tok = self._hist.gather(1, (self._step - 1).expand(self._hist.shape[0], 1))
        p, slot, ctx = self._decode_positions()
        md = AttentionMetadata(context_lens=ctx, kv_block_tables=self._bt,
                               slot_mapping=slot.unsqueeze(1), k_cache=self.pool.k_cache,
                               v_cache=self.pool.v_cache, k_scale=self.pool.k_scale,
                               v_scale=self.pool.v_scale, is_prefill=False,
                               decode_workspace=self._ws)
        logits = self.model(tok, p.unsqueeze(1), None, md, self._zero)
        nxt = torch.argmax(logits, dim=-1, keepdim=True)
        self._hist.scatter_(1, self._step.expand(self._hist.shape[0], 1), nxt)
        self._step += 1


@dataclass
class StepEntry:
    """One sequence's part of a step: ``n`` tokens from position ``start``; a decode
    feeds the token it sampled last; ``sample`` is the index of the token the step
    samples for it (None: a chunk that does not finish the prompt)."""

    sid: int
    start: int
    n: int
    decode: bool
    sample: Optional[int]


class ChunkedScheduler:
    """Host-side plan of continuous batching with chunked prefill (lengths only).

    Each step takes one token from every decoding sequence first, then prefill
    chunks of at most ``chunk`` tokens from sequences still reading their prompt,
    in admission order, up to ``max_step_tokens`` in all; waiting prompts are
    admitted (``admit(sid)`` is called) while the step has room.  A chunk that
    ends its prompt samples the first token; a sequence leaves after
    ``max_new`` tokens (``leave(sid)``).
    """

    def __init__(self, prompt_lens: List[int], max_new: int, max_step_tokens: int, chunk: int,
                 admit=None, leave=None):
        if max_new < 1 or chunk < 1 or max_step_tokens < 1:
            raise ValueError("max_new, chunk and max_step_tokens must be positive")
        self.lens = list(prompt_lens)
        self.max_new = max_new
        self.max_step_tokens = max_step_tokens
        self.chunk = chunk
        self.admit = admit or (lambda sid: None)
        self.leave = leave or (lambda sid: None)
        self.waiting = deque(range(len(self.lens)))
        self.filling: List[int] = []
        self.decoding: List[int] = []
        self.cached = [0] * len(self.lens)
        self.produced = [0] * len(self.lens)

    def done(self) -> bool:
        return not (self.waiting or self.filling or self.decoding)

    def _next_chunk(self, sid: int, budget: int) -> int:
        return min(self.chunk, self.lens[sid] - self.cached[sid], budget)

    def plan(self) -> List[StepEntry]:
        room = self.max_step_tokens - len(self.decoding) - sum(
            self._next_chunk(sid, self.max_step_tokens) for sid in self.filling)
        while self.waiting and room > 0:
            sid = self.waiting.popleft()
            self.admit(sid)
            self.filling.append(sid)
            room -= self._next_chunk(sid, self.max_step_tokens)
        out = [StepEntry(sid, self.lens[sid] + self.produced[sid] - 1, 1, True,
                         self.produced[sid]) for sid in self.decoding]
        budget = self.max_step_tokens - len(self.decoding)
        for sid in self.filling:
            if budget <= 0:
                break
            n = self._next_chunk(sid, budget)
            ends = self.cached[sid] + n == self.lens[sid]
            out.append(StepEntry(sid, self.cached[sid], n, False, 0 if ends else None))
            budget -= n
        return out

    def commit(self, step: List[StepEntry]) -> None:
        for e in step:
            if e.decode:
                self.produced[e.sid] += 1
            else:
                self.cached[e.sid] += e.n
                if self.cached[e.sid] == self.lens[e.sid]:
                    self.produced[e.sid] = 1
        still = []
        for sid in self.decoding:
            (self.leave(sid) if self.produced[sid] >= self.max_new else still.append(sid))
        for sid in [sid for sid in self.filling if self.cached[sid] == self.lens[sid]]:
            self.filling.remove(sid)
            (self.leave(sid) if self.produced[sid] >= self.max_new else still.append(sid))
        self.decoding = still


class MixedGenerator:
    """Continuous batching with chunked prefill over the attention path: each step
    of ``ChunkedScheduler`` runs as one packed row of tokens, decodes first, with
    ``PackedAttentionMetadata`` (one decode launch for the decode rows, one
    chunked-prefill launch over the paged cache for the chunk rows).

    A step's metadata is one descriptor upload expanded on the device
    (``nia_step_metadata_packed``).  Sampled tokens stay on the device and the next
    step reads them from there, so no step waits for the host.  Once no prompt is
    left to read, the remaining decode steps replay one captured HIP graph.
    Stats: ``prefill_steps`` counts the packed steps (mixed or not), ``prefill_s``
    the time until every prompt is in the cache.
    """

    def __init__(self, model: Qwen3ForCausalLM, pool: KVPool, max_new_tokens: int,
                 max_step_tokens: int = 8192, chunk: int = 1024, use_graph: bool = True):
        self.model = model
        self.pool = pool
        self.max_new = max_new_tokens
        self.max_step_tokens = max_step_tokens
        self.chunk = chunk
        self.use_graph = use_graph
        self.replay_hook = None  # called after every graph replay (tests interleave work)
        self.device = pool.k_cache.device

    def _decode_tail(self, sched: "ChunkedScheduler", host_blocks, prompts, st) -> None:
        """Once every sequence decodes, the remaining steps have one shape: feed each
        sequence's last token, sample the next.  They run as replays of one captured
        HIP graph; a sequence that has its max_new tokens keeps recomputing its last
        position (same slot, same values) and writes its sample to a spare entry."""
        import numpy as np

        dev = self.device
        sids = list(sched.decoding)
        b = len(sids)
        left = max(self.max_new - sched.produced[sid] for sid in sids)
        width = max(len(host_blocks[sid]) for sid in sids)
        bt = np.zeros((b, width), dtype=np.int32)
        for i, sid in enumerate(sids):
            bt[i, :len(host_blocks[sid])] = host_blocks[sid]
        self._bt = torch.from_numpy(bt).to(dev)
        self._sid = torch.tensor(sids, dtype=torch.int64, device=dev)
        self._plen = torch.tensor([len(prompts[sid]) for sid in sids], dtype=torch.int64,
                                  device=dev)
        self._prod = torch.tensor([sched.produced[sid] for sid in sids], dtype=torch.int64,
                                  device=dev)
        self._rows = torch.arange(b, device=dev)
        self._zero = torch.zeros(b, dtype=torch.int64, device=dev)
        self._spare = torch.full((b,), self._tok.numel() - 1, dtype=torch.int64, device=dev)
        self._ws = _graph_workspace(self.model, self.pool, self._bt)
        self._tail_step()
        st.decode_steps += 1
        if left > 1:
            if self.use_graph and left > 2:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    self._tail_step()
                for _ in range(left - 1):
                    graph.replay()
                    st.decode_steps += 1
                    if self.replay_hook is not None:
                        self.replay_hook()
            else:
                for _ in range(left - 1):
                    self._tail_step()
                    st.decode_steps += 1
        for sid in sids:
            sched.produced[sid] = self.max_new
            sched.leave(sid)
        sched.decoding = []

    def _tail_step(self) -> None:
        bs = self.pool.block_size
        last = self._prod - 1
        p = self._plen + last
        tok = self._tok[self._sid * self.max_new + last]
        slot = self._bt[self._rows, p // bs].to(torch.int64) * bs + p % bs
        md = AttentionMetadata(context_lens=p + 1, kv_block_tables=self._bt,
                               slot_mapping=slot.unsqueeze(1), k_cache=self.pool.k_cache,
                               v_cache=self.pool.v_cache, k_scale=self.pool.k_scale,
                               v_scale=self.pool.v_scale, is_prefill=False,
                               decode_workspace=self._ws)
        logits = self.model(tok.unsqueeze(1), p.unsqueeze(1), None, md, self._zero)
        live = self._prod < self.max_new
        dst = torch.where(live, self._sid * self.max_new + self._prod, self._spare)
        self._tok.index_put_((dst,), torch.argmax(logits, dim=-1))
        self._prod += live.to(torch.int64)

    @torch.no_grad()
    def run(self, prompts: List[List[int]]) -> GenerationStats:
        import numpy as np

        from . import _lib

        st = GenerationStats(prompt_tokens=sum(len(p) for p in prompts))
        dev = self.device
        n_seq = len(prompts)
        # one spare entry at the end takes the samples of finished sequences
        self._tok = torch.zeros(n_seq * self.max_new + 1, dtype=torch.int64, device=dev)
        blocks: Dict[int, List[int]] = {}
        host_blocks: Dict[int, np.ndarray] = {}

        def admit(sid):
            blocks[sid] = self.pool.allocate(len(prompts[sid]) + self.max_new)
            host_blocks[sid] = np.asarray(blocks[sid], dtype=np.int64)

        def leave(sid):
            self.pool.release(blocks.pop(sid))

        sched = ChunkedScheduler([len(p) for p in prompts], self.max_new, self.max_step_tokens,
                                 self.chunk, admit, leave)
        lib = _lib.load()
        stream = torch.cuda.current_stream(dev).cuda_stream
        bs = self.pool.block_size
        i64 = dict(dtype=torch.int64, device=dev)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        t1 = None
        while not sched.done():
            if not sched.waiting and not sched.filling:
                if t1 is None:
                    torch.cuda.synchronize(dev)
                    t1 = time.perf_counter()
                self._decode_tail(sched, host_blocks, prompts, st)
                break
            step = sched.plan()
            b, t = len(step), sum(e.n for e in step)
            nd = sum(1 for e in step if e.decode)
            hdr = np.zeros((b, 8), dtype=np.int64)
            host_tok, tables_h = [], []
            sample_row, sample_slot = [], []
            tok_off = blk_off = out_off = 0
            for i, e in enumerate(step):
                bl = host_blocks[e.sid]
                src = e.sid * self.max_new + e.sample - 1 if e.decode else -1
                hdr[i] = (e.n, e.start, len(bl), tok_off, blk_off, out_off, src, 0)
                if not e.decode:
                    host_tok.append(np.asarray(prompts[e.sid][e.start:e.start + e.n],
                                               dtype=np.int64))
                    tok_off += e.n
                tables_h.append(bl)
                blk_off += len(bl)
                out_off += e.n
                if e.sample is not None:
                    sample_row.append(i)
                    sample_slot.append(e.sid * self.max_new + e.sample)
            ns = len(sample_row)
            desc = np.concatenate([hdr.reshape(-1)] + host_tok + tables_h +
                                  [np.asarray(sample_row + sample_slot, dtype=np.int64)])
            d = torch.from_numpy(desc).pin_memory().to(dev, non_blocking=True)
            max_blocks = max(len(x) for x in tables_h)
            max_step = max(e.n for e in step)
            ids, pos, slots = (torch.empty(t, **i64) for _ in range(3))
            ctx, last = torch.empty(b, **i64), torch.empty(b, **i64)
            q_start = torch.empty(b, dtype=torch.int32, device=dev)
            q_len = torch.empty(b, dtype=torch.int32, device=dev)
            tables = torch.empty((b, max_blocks), dtype=torch.int32, device=dev)
            rc = lib.nia_step_metadata_packed(
                d.data_ptr(), tok_off, blk_off, self._tok.data_ptr(), self._tok.numel(), b, t,
                max_step, max_blocks, bs, ids.data_ptr(), pos.data_ptr(), slots.data_ptr(),
                ctx.data_ptr(), last.data_ptr(), q_start.data_ptr(), q_len.data_ptr(),
                tables.data_ptr(), stream)
            _lib.check("nia_step_metadata_packed", rc)
            md = PackedAttentionMetadata(
                context_lens=ctx, kv_block_tables=tables, slot_mapping=slots.unsqueeze(0),
                k_cache=self.pool.k_cache, v_cache=self.pool.v_cache, k_scale=self.pool.k_scale,
                               v_scale=self.pool.v_scale, is_prefill=nd < b,
                q_start=q_start, q_len=q_len, num_decode=nd,
                max_q_len=max((e.n for e in step[nd:]), default=1))
            tail = d[desc.size - 2 * ns:]
            logits = self.model.forward_packed(ids, pos, md, last[tail[:ns]])
            if ns:
                self._tok[tail[ns:]] = torch.argmax(logits, dim=-1)
            sched.commit(step)
            st.prefill_steps += 1
        torch.cuda.synchronize(dev)
        t2 = time.perf_counter()
        t1 = t2 if t1 is None else t1
        st.generated_tokens = n_seq * self.max_new
        st.prefill_s, st.decode_s, st.total_s = t1 - t0, t2 - t1, t2 - t0
        out = self._tok[:n_seq * self.max_new].view(n_seq, self.max_new).cpu()
        self.outputs = [out[i].tolist() for i in range(n_seq)]
        return st


def generation_prompts(num_requests: int = 64, lo: int = 128, hi: int = 2048,
                       vocab: int = 151936, seed: int = 4004) -> List[List[int]]:
    """64 prompts of U[128, 2048] token ids drawn U[0, vocab), seeded."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (num_requests,), generator=g).tolist()
    return [torch.randint(0, vocab, (n,), generator=g).tolist() for n in lens]


def build(cfg: Optional[Qwen3Config] = None, prompts: Optional[List[List[int]]] = None,
          max_new_tokens: int = 256, block_size: int = 16, max_prefill_batch: int = 8,
          device: str = "cuda", dtype=torch.bfloat16, seed: int = 4004,
          use_graph: bool = False, mixed: bool = False, max_step_tokens: int = 8192,
          chunk: int = 1024, fp8_cache: bool = False):
    """Random-initialised model, a KV pool sized for the prompts, and a generator:
    ``MixedGenerator`` (chunked prefill mixed with decodes) when ``mixed``, else the
    prefill-first ``Generator``; ``fp8_cache`` keeps the KV pool in the fp8 format."""
    cfg = cfg or Qwen3Config()
    prompts = prompts if prompts is not None else generation_prompts(seed=seed)
    model = Qwen3ForCausalLM(cfg).init_random(seed).to(device=device, dtype=dtype).eval()
    need = sum(math.ceil((len(p) + max_new_tokens) / block_size) for p in prompts)
    pool = KVPool(cfg, need + 16, block_size, dtype, torch.device(device), fp8=fp8_cache)
    if mixed:
        gen = MixedGenerator(model, pool, max_new_tokens, max_step_tokens, chunk,
                             use_graph=use_graph)
    else:
        gen = Generator(model, pool, max_new_tokens, max_prefill_batch, use_graph=use_graph)
    gen.prompts = prompts
    return gen


class AttentionTimer:
    """Context manager: HIP-event timing of every attention-path call (KV write, decode,
    prefill, chunked prefill) made through ``ops`` while active, and of every model
    forward, to report the attention path's share of the step time."""

    _NAMES = ("kv_write", "paged_decode", "prefill", "prefill_paged")

    def __init__(self, model: Qwen3ForCausalLM):
        self.model = model
        self.attn: List = []
        self.steps: List = []

    def _wrap(self, fn, sink):
        def timed(*args, **kwargs):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            r = fn(*args, **kwargs)
            b.record()
            sink.append((a, b))
            return r
        return timed

    def __enter__(self):
        self._saved = {n: getattr(ops, n) for n in self._NAMES}
        for n in self._NAMES:
            setattr(ops, n, self._wrap(self._saved[n], self.attn))
        self._fwd = self.model.forward
        self.model.forward = self._wrap(self._fwd, self.steps)
        return self

    def __exit__(self, *exc):
        for n, fn in self._saved.items():
            setattr(ops, n, fn)
        self.model.forward = self._fwd
        return False

    def totals_ms(self) -> Dict[str, float]:
        torch.cuda.synchronize()
        attn = sum(a.elapsed_time(b) for a, b in self.attn)
        steps = sum(a.elapsed_time(b) for a, b in self.steps)
        return {"attention_ms": attn, "step_ms": steps,
                "attention_share": attn / steps if steps > 0 else 0.0}


class HostTimer:
    """Context manager: host time (perf_counter) of every call made through the ``ops``
    wrappers while active.  That is what a call costs the CPU - validation, argument
    marshalling and the kernel launches - not the kernels, which run after the call has
    returned.  The wrapping itself adds two clock reads per call."""

    _NAMES = ("kv_write", "qk_norm_rope_kv_write", "paged_decode", "prefill", "prefill_paged")

    def __init__(self):
        self.calls: Dict[str, List[float]] = {n: [0, 0.0] for n in self._NAMES}

    def _wrap(self, name, fn):
        acc = self.calls[name]
        clock = time.perf_counter

        def timed(*args, **kwargs):
            t0 = clock()
            r = fn(*args, **kwargs)
            acc[1] += clock() - t0
            acc[0] += 1
            return r
        return timed

    def __enter__(self):
        self._saved = {n: getattr(ops, n) for n in self._NAMES}
        for n in self._NAMES:
            setattr(ops, n, self._wrap(n, self._saved[n]))
        return self

    def __exit__(self, *exc):
        for n, fn in self._saved.items():
            setattr(ops, n, fn)
        return False

    def per_call_us(self) -> Dict[str, Dict[str, float]]:
        return {n: {"calls": int(c), "host_us_per_call": round(t / c * 1e6, 2)}
                for n, (c, t) in self.calls.items() if c}


def main() -> int:
    import argparse
    import json

    ap = argparse.ArgumentParser(description="Qwen3-0.6B-architecture generation throughput")
    ap.add_argument("--requests", type=int, default=64)
    ap.add_argument("--max-new-tokens", type=int, default=256)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--prefill-batch", type=int, default=8)
    ap.add_argument("--time-attention", action="store_true")
    ap.add_argument("--eager", action="store_true", help="no HIP graph for the decode step")
    ap.add_argument("--mixed", action="store_true",
                    help="continuous batching with chunked prefill mixed with decodes")
    ap.add_argument("--step-tokens", type=int, default=8192)
    ap.add_argument("--chunk", type=int, default=1024)
    ap.add_argument("--fp8-cache", action="store_true", help="KV pool in the fp8 format")
    args = ap.parse_args()
    cfg = Qwen3Config(num_layers=args.layers)
    gen = build(cfg, generation_prompts(args.requests), args.max_new_tokens,
                max_prefill_batch=args.prefill_batch, use_graph=not args.eager,
                mixed=args.mixed, max_step_tokens=args.step_tokens, chunk=args.chunk,
                fp8_cache=args.fp8_cache)
    gen.run([p[:64] for p in gen.prompts[:4]])  # warm-up: kernels, allocator, workspaces
    st = gen.run(gen.prompts)
    line = {"tokens_per_s": round(st.tokens_per_s, 1),
            "decode_tokens_per_s": round(st.decode_tokens_per_s, 1),
            "prompt_tokens": st.prompt_tokens, "generated_tokens": st.generated_tokens,
            "prefill_s": round(st.prefill_s, 4), "decode_s": round(st.decode_s, 4),
            "total_s": round(st.total_s, 4), "prefill_steps": st.prefill_steps,
            "decode_steps": st.decode_steps}
    if args.time_attention:  # eager, so that every call is timed on its own
        gen.use_graph = False  # (the mixed generator has no graph)
        with AttentionTimer(gen.model) as tm:
            gen.run(gen.prompts)
        line.update({k: round(v, 4) for k, v in tm.totals_ms().items()})
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
