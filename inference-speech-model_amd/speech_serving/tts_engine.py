"""Streaming multi-codebook TTS engine on the paged KV kernels.

Same API as the reference's StreamingTTSEngine (speech_serving/tts_engine.py:
TTSRequest :25-45, engine :48-249): submit / step / run_until_done with
continuous batching over a BlockManager, prompt prefill, one multi-codebook frame
per step and request, per-frame streaming callbacks, blocks freed on completion.

Where the reference, per request and per step, gathers every layer's history out
of the pool into a contiguous cache (:166-185), runs the model on that request
alone, scatters the new K/V back (:191-198) and takes a torch.argmax per codebook
(:202), a step here is one batched pass over all active requests: per layer one
fused launch appends each request's new K/V through its block table and attends
over its paged history, and one argmax launch covers every (request, codebook)
row. The prompt prefill writes the prompt's K/V into the pool the same way (the
paged kernel's multi-token append with the causal mask).

Bookkeeping is the reference's: ceil(prompt_len / block_size) blocks at admission,
one more whenever the sequence length reaches a block boundary before a step,
all of a request's blocks freed when it completes or fails.

graph_decode (default on): each active request keeps a fixed slot; the decode step
of a batch bucket (the smallest of 1, 2, 4, ... covering the highest busy slot)
is captured once in a HIP graph over static per-slot buffers (input frame, block
table, length, output tokens) and replayed every step: the graph runs the layers,
the argmax into the slot tokens and the copy of those tokens into the next step's
input frames, so a step's host work is two small uploads (lengths, changed table
rows) and one replay. Idle slots have length 0: their attention launches return
at once and append nothing. The context cap of the captured graphs doubles when a
request outgrows it (the graphs are captured again).
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Tuple

import torch

from . import native
from .block_manager import BlockManager
from .models import KVCache, LayerKV, PagedKV, PagedKVCache, StreamingMultiCodebookTTSModel


@dataclass
class TTSRequest:
    """A streaming TTS generation request (reference tts_engine.py:25-45)."""
    id: int
    prompt_codebooks: torch.Tensor  # [seq_len, num_codebooks]
    max_new_frames: int
    arrival_time: float = 0.0

    seq_len: int = 0
    block_table: List[int] = field(default_factory=list)
    generated_frames: List[torch.Tensor] = field(default_factory=list)  # [num_codebooks] each
    generated_count: int = 0
    done: bool = False

    start_time: Optional[float] = None
    first_token_time: Optional[float] = None
    last_frame_codebooks: Optional[torch.Tensor] = None  # [1, 1, num_codebooks]
    on_frame_callback: Optional[Callable[[int, torch.Tensor], None]] = None


class StreamingTTSEngine:
    """Continuous batching of streaming multi-codebook TTS requests over a paged KV pool."""

    def __init__(self, model: StreamingMultiCodebookTTSModel, block_manager: BlockManager, max_batch_size: int = 8,
                 device: str = "cuda", graph_decode: Optional[bool] = None):
        self.model = model
        self.block_manager = block_manager
        self.max_batch_size = max_batch_size
        self.device = device
        # The model is called as the reference calls it, model(input_codebooks, past_key_values, use_cache)
        # (tts_engine.py:188): models with the paged step get a PagedKVCache; a model with only that
        # forward is served on K/V gathered from the pool, one request at a time, as the reference does.
        self._paged_model = callable(getattr(model, "decode_step_paged", None))
        if graph_decode is None:
            graph_decode = self._paged_model
        if graph_decode and not self._paged_model:
            raise TypeError(f"graph decode captures the model's paged step (decode_step_paged); "
                            f"{type(model).__name__} has none: use graph_decode=False")
        self.graph_decode = graph_decode

        self.active: List[TTSRequest] = []
        self.queue: List[TTSRequest] = []
        self.completed: List[TTSRequest] = []
        self._next_id = 0

        # graph decode state (allocated on first use)
        self._slot_of: Dict[int, int] = {}  # request id -> slot
        self._free_slots = list(range(max_batch_size))
        self._cap = 0  # context cap (tokens) of the captured graphs and the table width
        self._graphs: Dict[int, torch.cuda.CUDAGraph] = {}
        self._graph_pool = None
        self._graph_workspaces: List[torch.Tensor] = []  # attention workspaces the graphs were captured with

    # -- API -------------------------------------------------------------------
    def submit(self, prompt_codebooks: torch.Tensor, max_new_frames: int = 100, arrival_time: float = 0.0,
               on_frame_callback: Optional[Callable[[int, torch.Tensor], None]] = None) -> int:
        """Queue a request: prompt_codebooks [prompt_len, num_codebooks], up to max_new_frames frames."""
        req = TTSRequest(id=self._next_id, prompt_codebooks=prompt_codebooks.to(self.device),
                         max_new_frames=max_new_frames, arrival_time=arrival_time,
                         on_frame_callback=on_frame_callback)
        self._next_id += 1
        self.queue.append(req)
        return req.id

    def step(self) -> bool:
        """Admit queued requests, then produce one frame for every active request."""
        self._admit_from_queue()
        if not self.active:
            return False
        bm = self.block_manager
        batch: List[TTSRequest] = []
        for req in self.active:
            try:
                if req.seq_len % bm.block_size == 0:
                    req.block_table.append(bm.allocate_block())
                batch.append(req)
            except Exception as e:  # out of blocks: this request ends, the others go on
                self._fail(req, e)
        still_active: List[TTSRequest] = []
        if batch:
            try:
                if self.graph_decode:
                    rows = self._decode_graph(batch)
                    frames = [rows[self._slot_of[r.id]] for r in batch]
                else:
                    frames = self._decode(batch)
            except Exception as e:
                for req in batch:
                    self._fail(req, e)
            else:
                for i, req in enumerate(batch):
                    req.seq_len += 1
                    if self._emit(req, frames[i]):
                        still_active.append(req)
        self.active = still_active
        return True

    def run_until_done(self, max_steps: int = 10000) -> List[TTSRequest]:
        """Step until the queue and the active set are empty (or max_steps)."""
        steps = 0
        while (self.active or self.queue) and steps < max_steps:
            if not self.step():
                break
            steps += 1
        return self.completed

    # -- internals ---------------------------------------------------------------
    def _admit_from_queue(self) -> None:
        bm = self.block_manager
        while len(self.active) < self.max_batch_size and self.queue:
            req = self.queue.pop(0)
            req.start_time = time.perf_counter()
            prompt_len = req.prompt_codebooks.shape[0]
            req.seq_len = prompt_len
            try:
                for _ in range((prompt_len + bm.block_size - 1) // bm.block_size):
                    req.block_table.append(bm.allocate_block())
                frame = self._prefill(req)
            except Exception:
                # As in the reference, an admission error propagates to the caller;
                # the request's blocks are returned first.
                bm.free_blocks(req.block_table)
                req.block_table = []
                raise
            req.first_token_time = time.perf_counter()
            if self._emit(req, frame):
                if self.graph_decode:
                    self._take_slot(req, frame)
                self.active.append(req)

    def _paged_cache(self, tables: List[List[int]], ctx: List[int]) -> PagedKVCache:
        bm = self.block_manager
        width = max(len(t) for t in tables)
        rows = [t + [0] * (width - len(t)) for t in tables]  # padding past a row's keys is never read
        dev = bm.key_pool[0].device
        return PagedKVCache(bm.key_pool, bm.value_pool, torch.tensor(rows, dtype=torch.int32).to(dev),
                            torch.tensor(ctx, dtype=torch.int32).to(dev), max(ctx),
                            rows_longest_first=all(a >= b for a, b in zip(ctx, ctx[1:])))

    @torch.no_grad()
    def _prefill(self, req: TTSRequest) -> torch.Tensor:
        """Prompt forward: its K/V go into the request's blocks; returns the first frame [K]."""
        codes = req.prompt_codebooks.unsqueeze(0)
        if self._paged_model:
            out = self.model(input_codebooks=codes, past_key_values=self._paged_cache([req.block_table],
                                                                                     [req.seq_len]),
                             use_cache=True, logits_to_keep=1)
        else:
            out = self.model(input_codebooks=codes, past_key_values=None, use_cache=True)
            self._append_kv(out.past_key_values, [req], 0, req.seq_len)
        return self._greedy(out.logits[:, -1])[0]

    @torch.no_grad()
    def _decode(self, batch: List[TTSRequest]) -> List[torch.Tensor]:
        """One frame for every request of the batch: [K] codebook tokens each."""
        if not self._paged_model:
            return [self._decode_contiguous(r) for r in batch]
        cache = self._paged_cache([r.block_table for r in batch], [r.seq_len + 1 for r in batch])
        inputs = torch.cat([r.last_frame_codebooks for r in batch], dim=0)  # [B, 1, K]
        out = self.model(input_codebooks=inputs, past_key_values=cache, use_cache=True, logits_to_keep=1)
        return list(self._greedy(out.logits[:, -1]).unbind(0))

    def _decode_contiguous(self, req: TTSRequest) -> torch.Tensor:
        """The reference's step for one request (tts_engine.py:174-204): its history gathered out of the
        pool (skv_gather), the model forward on that contiguous cache, the new frame's K/V appended into
        the pool (skv_append)."""
        bm = self.block_manager
        dev = bm.key_pool[0].device
        table = torch.tensor([req.block_table], dtype=torch.int32, device=dev)
        lens = torch.tensor([req.seq_len], dtype=torch.int32, device=dev)
        cache = KVCache([LayerKV(*native.gather(bm.key_pool[l], bm.value_pool[l], table, lens, req.seq_len))
                         for l in range(bm.num_layers)])
        out = self.model(input_codebooks=req.last_frame_codebooks, past_key_values=cache, use_cache=True)
        self._append_kv(out.past_key_values, [req], req.seq_len, 1)
        return self._greedy(out.logits[:, -1])[0]

    def _append_kv(self, cache, reqs: List[TTSRequest], start: int, n: int) -> None:
        """Append the last n positions of each layer's returned K/V ([B, H, T, D]) at positions
        start..start+n-1 of each request's blocks (the reference's block writes, :191-198)."""
        bm = self.block_manager
        dev = bm.key_pool[0].device
        slots = torch.tensor([bm.slot(r.block_table, start + i) for r in reqs for i in range(n)],
                             dtype=torch.int64).to(dev)
        for l in range(bm.num_layers):
            k, v = cache.layers[l].keys[:, :, -n:], cache.layers[l].values[:, :, -n:]
            rows = k.shape[0] * n
            native.append(k.permute(0, 2, 1, 3).reshape(rows, k.shape[1], k.shape[3]),
                          v.permute(0, 2, 1, 3).reshape(rows, v.shape[1], v.shape[3]),
                          bm.key_pool[l], bm.value_pool[l], slots)

    def _greedy(self, logits: torch.Tensor) -> torch.Tensor:
        """Argmax per (request, codebook) row of logits [B, K, V] -> int64 [B, K]."""
        b, k, v = logits.shape
        return native.argmax(logits.reshape(b * k, v)).view(b, k)

    # -- graph decode ------------------------------------------------------------
    def _buckets(self) -> List[int]:
        out, b = [], 1
        while b < self.max_batch_size:
            out.append(b)
            b *= 2
        return out + [self.max_batch_size]

    def _setup_graph_buffers(self, cap: int) -> None:
        """(Re)allocate the static slot buffers for a context cap; drops captured graphs."""
        bm = self.block_manager
        s, k = self.max_batch_size, self.model.num_codebooks
        width = -(-cap // bm.block_size)
        dev = bm.key_pool[0].device
        if self._graphs:
            torch.cuda.synchronize(dev)  # no replay of the graphs being dropped is still pending
        self._graphs.clear()
        self._graph_pool = None
        self._cap = width * bm.block_size
        self._width = width
        self.g_inputs = torch.zeros((s, 1, k), dtype=torch.int64, device=dev)
        # Per-slot metadata in one buffer (one upload per step): lengths [S], then tables [S, W].
        self.g_meta = torch.zeros(s + s * width, dtype=torch.int32, device=dev)
        self.g_ctx = self.g_meta[:s]
        self.g_tables = self.g_meta[s:].view(s, width)
        self.g_tokens = torch.zeros(s * k, dtype=torch.int64, device=dev)
        # Two pinned banks, each reused only after its previous upload has run; each bank
        # tracks how many table entries of every slot it holds.
        self._banks = [torch.zeros(s + s * width, dtype=torch.int32).pin_memory() for _ in range(2)]
        self._bank_events = [None, None]
        self._bank_filled = [[-1] * s, [-1] * s]
        self._bank_i = 0
        for r in self.active:
            self.g_inputs[self._slot_of[r.id]].copy_(r.last_frame_codebooks[0])
        self._graph_workspaces = []
        for b in self._buckets():
            native.reserve_attention(b, self.model.num_heads, self.model.head_dim, self._cap, self.model.dtype, dev)

    def _graph_step(self, inputs, tables, ctx, tokens, b: int) -> None:
        """The captured decode step of bucket b over the given slot buffers."""
        bm = self.block_manager
        k, v = self.model.num_codebooks, self.model.vocab_size
        kv = PagedKV(bm.key_pool, bm.value_pool, tables[:b], ctx[:b], self._cap)
        logits = self.model.decode_step_paged(inputs[:b], kv)  # [b, K, V]
        native.argmax(logits.reshape(b * k, v), out=tokens[:b * k])
        inputs[:b, 0].copy_(tokens[:b * k].view(b, k))

    def _graph_for(self, b: int) -> torch.cuda.CUDAGraph:
        g = self._graphs.get(b)
        if g is not None:
            return g
        dev = self.g_inputs.device
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.no_grad(), torch.cuda.stream(side):
            # Warm-up on throwaway buffers (all lengths 0, so nothing is appended): builds the
            # model's fused weights and the GEMM library state outside the capture.
            scratch = (torch.zeros_like(self.g_inputs), torch.zeros_like(self.g_tables),
                       torch.zeros_like(self.g_ctx), torch.zeros_like(self.g_tokens))
            self._graph_step(*scratch, b)
        torch.cuda.current_stream(dev).wait_stream(side)
        g = torch.cuda.CUDAGraph()
        kwargs = {"pool": self._graph_pool} if self._graph_pool is not None else {}
        with torch.no_grad(), torch.cuda.graph(g, stream=side, **kwargs):
            self._graph_step(self.g_inputs, self.g_tables, self.g_ctx, self.g_tokens, b)
        if self._graph_pool is None:
            self._graph_pool = g.pool()
        self._graphs[b] = g
        # The graph holds the attention workspace's address: keep that buffer alive even if a
        # later, larger call grows the device's workspace (which drops the old one).
        ws = native.reserve_workspace(0, dev)
        if all(w.data_ptr() != ws.data_ptr() for w in self._graph_workspaces):
            self._graph_workspaces.append(ws)
        return g

    def _decode_graph(self, batch: List[TTSRequest]) -> Tuple[torch.Tensor, ...]:
        """One frame for every request of the batch via the captured step; the [K] frame of slot i is
        element i of the returned tuple (views of one token tensor, made in one call)."""
        need = max(r.seq_len + 1 for r in batch)
        if need > self._cap:
            cap = max(256, self._cap)
            while cap < need:
                cap *= 2
            self._setup_graph_buffers(cap)
        top = max(self._slot_of[r.id] for r in batch) + 1
        b = next(x for x in self._buckets() if x >= top)
        i = self._bank_i
        self._bank_i ^= 1
        if self._bank_events[i] is not None:
            self._bank_events[i].synchronize()
        bank, filled, s = self._banks[i], self._bank_filled[i], self.max_batch_size
        host = bank.numpy()
        host[:s] = 0
        tables = host[s:].reshape(s, self._width)
        for r in batch:
            slot = self._slot_of[r.id]
            host[slot] = r.seq_len + 1
            n = len(r.block_table)
            if filled[slot] != n:
                tables[slot, :n] = r.block_table
                filled[slot] = n
        self.g_meta.copy_(bank, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._bank_events[i] = ev
        self._graph_for(b).replay()
        return self.g_tokens[:b * self.model.num_codebooks].view(b, -1).clone().unbind(0)

    def _take_slot(self, req: TTSRequest, frame: torch.Tensor) -> None:
        slot = self._free_slots.pop(0)
        self._slot_of[req.id] = slot
        if self._cap:
            for filled in self._bank_filled:
                filled[slot] = -1  # a new request's table: every bank rewrites the row
            self.g_inputs[slot, 0].copy_(frame)

    def _release_slot(self, req: TTSRequest) -> None:
        slot = self._slot_of.pop(req.id, None)
        if slot is not None:
            self._free_slots.append(slot)
            self._free_slots.sort()

    def _emit(self, req: TTSRequest, frame: torch.Tensor) -> bool:
        """Record one frame; returns whether the request stays active."""
        req.last_frame_codebooks = frame.view(1, 1, -1)
        req.generated_frames.append(frame)
        req.generated_count += 1
        if req.on_frame_callback is not None:
            try:
                req.on_frame_callback(req.id, frame)
            except Exception as e:
                print(f"Warning: Exception in frame callback for req {req.id}: {e}")
        if req.generated_count >= req.max_new_frames:
            self._finish(req)
            return False
        return True

    def _finish(self, req: TTSRequest) -> None:
        self._release_slot(req)
        req.done = True
        self.block_manager.free_blocks(req.block_table)
        req.block_table = []
        self.completed.append(req)

    def _fail(self, req: TTSRequest, err: Exception) -> None:
        print(f"Error executing step for TTS request {req.id}: {err}")
        self._finish(req)
