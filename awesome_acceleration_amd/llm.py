"""Continuous-batching Qwen3 engine on the gfx950 attention kernels.

Restates the reference's single-GPU engine (llm.py:36-446): an async request
queue served by a background loop that, each iteration, (1) drains the queue,
(2) admits waiting prompts while capacity lasts, (3) runs one packed varlen
prefill for the newly admitted prompts and samples their first token, (4)
runs one batched decode step for every active sequence, and (5) retires
finished sequences.  Finish rule (llm.py:371, :421-425): ``len(tokens) >=
max_tokens``, position ``>= max_seq_len``, or EOS unless ``ignore_eos``.
Greedy sampling at temperature 0 (llm.py:215-219).

Changes on the hot path:

* Capacity is a pool of fixed-size KV blocks (``BlockAllocator``) instead of
  one ``max_seq_len`` slot per sequence; a sequence is admitted when a batch
  row and the blocks for ``min(prompt + max_tokens, max_seq_len)`` tokens are
  free (so it can never run out of cache mid-generation).
* Per-step metadata (token ids, positions, cache lengths, block tables) is
  packed on the host and copied to the device once per step; the model has no
  per-layer host synchronisation (the reference syncs in RoPE,
  model/model.py:82, and writes decode inputs element by element,
  llm.py:395-398).
* With HIP graphs, a decode step of an unchanged batch is launched from the
  device-side state the previous step left (sampled ids as the next input,
  positions and cache lengths advanced in place) before the host reads the
  previous step's tokens, so the host's bookkeeping overlaps the GPU; the
  reference's loop syncs on every step's tokens (llm.py:404-405, :413-443).
* No tokenizer is available offline, so prompts are token-id lists and
  ``GenerationOutput.text`` is empty unless a ``decode_fn`` is supplied.
"""
from __future__ import annotations

import bisect
import concurrent.futures
import math
import queue
import threading
import time
from dataclasses import dataclass, field
from typing import Callable, Optional

import numpy as np
import torch

from . import fused as fz
from .paged import BlockAllocator, build_prefill_metadata, pad_block_tables
from .qwen3 import PagedKVCache, Qwen3Config, Qwen3ForCausalLM, StepMeta

__all__ = ["LLM", "GenerationOutput"]


@dataclass
class GenerationOutput:
    """Result of one prompt (llm.py:15-21)."""
    text: str
    token_ids: list[int]
    prompt_tokens: int = 0
    generated_tokens: int = 0


@dataclass
class _Request:
    """Internal request record (llm.py:24-33)."""
    token_ids: list[list[int]]
    max_tokens: int
    temperature: float
    ignore_eos: bool
    future: concurrent.futures.Future
    results: list = field(default_factory=list)
    pending_indices: list = field(default_factory=list)


@dataclass
class _Seq:
    req: _Request
    prompt_idx: int
    row: int                 # batch row (the reference's slot id)
    blocks: list[int]
    tokens: list[int]        # generated so far
    pos: int                 # position of the next token to feed
    done: bool = False       # finished (a step launched ahead may still hold its row)


class LLM:
    """Qwen3 engine with continuous batching and a paged KV cache.

    ``max_num_seqs`` bounds the decode batch (the reference's slot count);
    ``num_blocks`` defaults to enough blocks for ``max_num_seqs`` sequences
    of ``max_seq_len`` tokens.
    """

    def __init__(self, config: Optional[Qwen3Config] = None, max_num_seqs: int = 32,
                 max_seq_len: int = 4096, dtype=torch.bfloat16, block_size: int = 256,
                 num_blocks: Optional[int] = None, seed: int = 0, device="cuda",
                 decode_fn: Optional[Callable[[list[int]], str]] = None, use_graphs: bool = True,
                 fused: bool = True):
        self.device = torch.device(device)
        self.dtype = dtype
        self.config = config or Qwen3Config()
        self.max_seq_len = max_seq_len
        self.max_num_seqs = max_num_seqs
        self.block_size = block_size
        self.blocks_per_seq = math.ceil(max_seq_len / block_size)
        if num_blocks is None:
            num_blocks = max_num_seqs * self.blocks_per_seq
        self.decode_fn = decode_fn
        self.model = Qwen3ForCausalLM(self.config, self.device, dtype, seed, fused=fused)
        # block 0 is a scratch block: padding rows of a graph-captured decode
        # step append into it, so they never touch a live sequence's cache
        self.cache = PagedKVCache(self.config, num_blocks + 1, block_size, self.device, dtype)
        self.allocator = BlockAllocator(num_blocks + 1)
        self.allocator.allocate(1)
        self.use_graphs = use_graphs
        self._graphs: dict[int, tuple] = {}
        # packed per-step host metadata: ids | positions | seqlens | ctx | tables | live
        # (live = 1 for a sequence's row, 0 for a graph padding row)
        W = self.blocks_per_seq
        self._host = torch.zeros(max_num_seqs * (5 + W), dtype=torch.int32, pin_memory=True)
        self._dev = torch.zeros(max_num_seqs * (5 + W), dtype=torch.int32, device=self.device)
        # sampled ids of a decode step launched ahead, read back without a sync
        self._tok_host = [torch.zeros(max_num_seqs, dtype=torch.int32, pin_memory=True)
                          for _ in range(2)]
        self._tok_turn = 0
        self._request_queue: queue.Queue[_Request] = queue.Queue()
        self._loop_running = False
        self._loop_thread: Optional[threading.Thread] = None
        self.stats = dict(prefill_calls=0, decode_steps=0, prefill_tokens=0, decode_tokens=0)

    # ------------------------------------------------------------------ API
    def generate(self, prompts: list[list[int]], max_tokens: int = 100, temperature: float = 0.0,
                 ignore_eos: bool = False) -> concurrent.futures.Future:
        """Submit token-id prompts; the future resolves to ``list[GenerationOutput]``
        in prompt order (llm.py:225-264)."""
        if not prompts:
            raise ValueError("no prompts")
        pool = self.allocator.num_blocks - 1  # block 0 is the scratch block
        for p in prompts:
            if not p:
                raise ValueError("empty prompt")
            if len(p) >= self.max_seq_len:
                raise ValueError(f"prompt of {len(p)} tokens does not fit max_seq_len "
                                 f"{self.max_seq_len}")
            if self._blocks_for(len(p), max_tokens) > pool:
                # admission reserves every block a sequence can reach up front;
                # a request that needs more than the whole pool would wait forever
                raise ValueError(f"prompt of {len(p)} tokens with max_tokens {max_tokens} needs "
                                 f"{self._blocks_for(len(p), max_tokens)} KV blocks; the pool "
                                 f"has {pool}")
        self._ensure_loop()
        fut: concurrent.futures.Future = concurrent.futures.Future()
        req = _Request(token_ids=[list(map(int, p)) for p in prompts], max_tokens=max_tokens,
                       temperature=temperature, ignore_eos=ignore_eos, future=fut,
                       results=[None] * len(prompts), pending_indices=list(range(len(prompts))))
        self._request_queue.put(req)
        return fut

    def _blocks_for(self, prompt_len: int, max_tokens: int) -> int:
        """KV blocks reserved at admission: every position the sequence can reach."""
        return math.ceil(min(prompt_len + max_tokens, self.max_seq_len) / self.block_size)

    def stop(self, timeout: float = 30.0):
        """Stop the background loop (llm.py:302-309)."""
        if not self._loop_running:
            return
        self._loop_running = False
        if self._loop_thread:
            self._loop_thread.join(timeout=timeout)
            self._loop_thread = None

    def _ensure_loop(self):
        if not self._loop_running:
            self._loop_running = True
            self._loop_thread = threading.Thread(target=self._inference_loop, daemon=True)
            self._loop_thread.start()

    # ------------------------------------------------------------ core steps
    def _sample(self, logits: torch.Tensor, temperature: float) -> list[int]:
        if temperature == 0:
            return fz.argmax(logits).tolist()
        probs = torch.softmax(logits.float() / temperature, dim=-1)
        return torch.multinomial(probs, 1).squeeze(-1).tolist()

    def _prefill(self, seqs: list[_Seq]) -> torch.Tensor:
        """Packed varlen prefill of newly admitted sequences (llm.py:116-208)."""
        prompts = [s.req.token_ids[s.prompt_idx] for s in seqs]
        lens = [len(p) for p in prompts]
        tables = pad_block_tables([s.blocks for s in seqs], self.blocks_per_seq)
        # a slot outside the cache raises IndexError here, before any launch,
        # as the reference's index_copy_ store does (llm.py:171-174)
        cu, positions, slots = build_prefill_metadata(
            lens, tables, self.block_size, self.device,
            num_cache_rows=self.cache.num_blocks * self.block_size)
        ids = torch.from_numpy(np.fromiter((t for p in prompts for t in p), dtype=np.int64,
                                           count=sum(lens))).to(self.device)
        last = (cu[1:] - 1).long()
        meta = StepMeta(positions=positions, cu_seqlens=cu, slot_mapping=slots,
                        max_seqlen=max(lens), last_idx=last)
        self.stats["prefill_calls"] += 1
        self.stats["prefill_tokens"] += sum(lens)
        return self.model.forward(ids, meta, self.cache, prefill=True)

    def _decode_meta(self, B: int, max_context_len: int) -> StepMeta:
        d, W = self._dev, self.blocks_per_seq
        return StepMeta(positions=d[B:2 * B], cache_seqlens=d[2 * B:3 * B],
                        context_lens=d[3 * B:4 * B],
                        block_tables=d[4 * B:4 * B + B * W].view(B, W),
                        max_context_len=max_context_len)

    def _decode_step(self, seqs: list[_Seq]) -> torch.Tensor:
        """One token for every active sequence (llm.py:210-213, model/model.py:233-241).

        With graphs enabled the batch is padded to a power-of-two bucket and
        the captured step of that bucket is replayed; padding rows append to
        the scratch block 0 at position 0 and their logits are dropped.
        """
        n, W = len(seqs), self.blocks_per_seq
        B = self._bucket(n)
        h = self._host.numpy()
        h[:5 * B + B * W] = 0
        h[:n] = [s.tokens[-1] for s in seqs]
        h[B:B + n] = [s.pos for s in seqs]
        h[2 * B:2 * B + n] = h[B:B + n]              # tokens already in the cache
        h[3 * B:4 * B] = h[2 * B:3 * B] + 1           # context after the append
        tab = h[4 * B:4 * B + B * W].reshape(B, W)
        for i, s in enumerate(seqs):
            tab[i, :len(s.blocks)] = s.blocks
        # every sequence's append row must be a row of its own blocks (the
        # error the reference's store raises for a bad index, llm.py:171-174);
        # padding rows append into the scratch block 0
        if (int(tab[:n].max(initial=0)) >= self.cache.num_blocks or int(tab[:n].min(initial=0)) < 0
                or any(s.pos >= len(s.blocks) * self.block_size for s in seqs)):
            raise IndexError(f"decode append outside the KV cache ({self.cache.num_blocks} blocks "
                             f"of {self.block_size})")
        h[4 * B + B * W:4 * B + B * W + n] = 1        # live rows
        m = B * (5 + W)
        self._dev[:m].copy_(self._host[:m], non_blocking=True)
        self.stats["decode_steps"] += 1
        if not self.use_graphs:
            meta = self._decode_meta(B, self.blocks_per_seq * self.block_size)
            return self.model.forward(self._dev[:B], meta, self.cache, prefill=False)
        g = self._graphs.get(B)
        if g is None:
            g = self._capture(B)
        g[0].replay()
        return g[1][:n]

    def _bucket(self, n: int) -> int:
        return min(1 << (n - 1).bit_length(), self.max_num_seqs) if self.use_graphs else n

    def _sample_ahead(self, n: int, temperature: float):
        """After a graph step of n sequences: sample every row on the device,
        make the samples the next step's input ids, advance the live rows'
        positions and cache lengths by one (the device-side state of the
        next step, whose block tables are unchanged: blocks are reserved at
        admission), and copy the samples to pinned host memory.  Returns the
        handle ``_tokens`` waits on."""
        B, W = self._bucket(n), self.blocks_per_seq
        logits = self._graphs[B][1]
        if temperature == 0:
            tok = fz.argmax(logits)
        else:
            tok = torch.multinomial(torch.softmax(logits.float() / temperature, dim=-1), 1)
            tok = tok.squeeze(-1)
        d = self._dev
        d[:B].copy_(tok)
        d[B:4 * B].view(3, B).add_(d[4 * B + B * W:5 * B + B * W].view(1, B))
        buf = self._tok_host[self._tok_turn]
        self._tok_turn ^= 1
        buf[:B].copy_(d[:B], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        return n, ev, buf

    def _step_ahead(self, n: int):
        """Replay the graph of the last batch from the device-side state."""
        self.stats["decode_steps"] += 1
        self._graphs[self._bucket(n)][0].replay()

    @staticmethod
    def _tokens(handle) -> list[int]:
        n, ev, buf = handle
        ev.synchronize()
        return buf[:n].tolist()

    def _capture(self, B: int):
        """Capture one decode step of batch B as a HIP graph.  Every launch
        reads its inputs from the static metadata buffer; the attention grid
        is sized by the block-table capacity, so the graph is valid for every
        step of this bucket."""
        meta = self._decode_meta(B, self.blocks_per_seq * self.block_size)
        ids = self._dev[:B]
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for _ in range(2):  # warm up: workspace and allocator pools
                self.model.forward(ids, meta, self.cache, prefill=False)
        torch.cuda.current_stream(self.device).wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = self.model.forward(ids, meta, self.cache, prefill=False)
        self._graphs[B] = (graph, logits)
        return self._graphs[B]

    # ------------------------------------------------------------ the loop
    def _finish(self, s: _Seq, free_rows: list[int]):
        req = s.req
        s.done = True
        text = self.decode_fn(s.tokens) if self.decode_fn else ""
        req.results[s.prompt_idx] = GenerationOutput(
            text, list(s.tokens), len(req.token_ids[s.prompt_idx]), len(s.tokens))
        self.allocator.free(s.blocks)
        bisect.insort(free_rows, s.row)
        if all(r is not None for r in req.results):
            req.future.set_result(req.results)

    def _retire(self, seqs: list[_Seq], sampled: list[int], active: dict, free_rows: list[int]) -> bool:
        """Phase 5 for one decode step: append each live sequence's token and
        finish those that stop.  Returns whether any sequence finished."""
        finished = False
        for s, tok in zip(seqs, sampled):
            if s.done:  # finished after an earlier step; this row's token is dropped
                continue
            s.tokens.append(tok)
            s.pos += 1
            self.stats["decode_tokens"] += 1
            if self._should_stop(s, tok):
                del active[s.row]
                self._finish(s, free_rows)
                finished = True
        return finished

    def _should_stop(self, s: _Seq, tok: int) -> bool:
        return (len(s.tokens) >= s.req.max_tokens or s.pos >= self.max_seq_len
                or (not s.req.ignore_eos and tok == self.config.eos_token_id))

    @torch.inference_mode()
    def _inference_loop(self):
        free_rows = list(range(self.max_num_seqs))
        active: dict[int, _Seq] = {}
        pending: list[_Request] = []
        try:
            while self._loop_running or pending or active:
                # Phase 1: drain the queue
                while True:
                    try:
                        pending.append(self._request_queue.get_nowait())
                    except queue.Empty:
                        break
                if not pending and not active:
                    if not self._loop_running:
                        break
                    time.sleep(0.001)
                    continue
                # Phase 2: admit while a batch row and the blocks are free
                new: list[_Seq] = []
                for req in list(pending):
                    while req.pending_indices and free_rows:
                        pi = req.pending_indices[0]
                        L = len(req.token_ids[pi])
                        need = self._blocks_for(L, req.max_tokens)
                        if need > self.allocator.num_free:
                            break
                        req.pending_indices.pop(0)
                        new.append(_Seq(req, pi, free_rows.pop(0), self.allocator.allocate(need),
                                        [], L))
                    if not req.pending_indices:
                        pending.remove(req)
                    elif not free_rows or self.allocator.num_free == 0:
                        break
                # Phase 3: prefill the admitted prompts, sample their first token
                if new:
                    sampled = self._sample(self._prefill(new), new[0].req.temperature)
                    for s, tok in zip(new, sampled):
                        s.tokens.append(tok)
                        if 1 >= s.req.max_tokens or (not s.req.ignore_eos
                                                     and tok == self.config.eos_token_id):
                            self._finish(s, free_rows)
                        else:
                            active[s.row] = s
                if not active:
                    continue
                # Phase 4: one decode step for every active sequence
                seqs = [active[r] for r in sorted(active)]
                temp = seqs[0].req.temperature
                if not self.use_graphs:
                    self._retire(seqs, self._sample(self._decode_step(seqs), temp), active,
                                 free_rows)  # Phase 5: bookkeeping
                    continue
                # With graphs the next step of the same batch is launched from
                # the device-side state before the host reads this step's
                # tokens, so the bookkeeping and the next launch overlap the
                # GPU.  A row that finishes computes one discarded token in
                # the step launched ahead (into its own blocks, before they
                # can be handed to a later prefill on the same stream); the
                # batch is rebuilt on the host once rows finish or a waiting
                # request may be admitted.
                self._decode_step(seqs)
                h = self._sample_ahead(len(seqs), temp)
                while True:
                    ahead = None
                    if self._request_queue.empty() and (not pending or not free_rows):
                        self._step_ahead(len(seqs))
                        ahead = self._sample_ahead(len(seqs), temp)
                    finished = self._retire(seqs, self._tokens(h), active, free_rows)
                    if ahead is None:
                        break
                    h = ahead
                    if finished or not self._loop_running:
                        self._retire(seqs, self._tokens(h), active, free_rows)
                        break
        except BaseException as e:  # surface failures to every waiting caller
            for s in active.values():
                if not s.req.future.done():
                    s.req.future.set_exception(e)
            for req in pending:
                if not req.future.done():
                    req.future.set_exception(e)
            while True:
                try:
                    req = self._request_queue.get_nowait()
                except queue.Empty:
                    break
                if not req.future.done():
                    req.future.set_exception(e)
            self._loop_running = False
            raise
