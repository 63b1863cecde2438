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
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional

import torch

from . import native
from .block_manager import BlockManager
from .models import PagedKV, StreamingMultiCodebookTTSModel


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
                 device: str = "cuda"):
        self.model = model
        self.block_manager = block_manager
        self.max_batch_size = max_batch_size
        self.device = device

        self.active: List[TTSRequest] = []
        self.queue: List[TTSRequest] = []
        self.completed: List[TTSRequest] = []
        self._next_id = 0

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
                self.active.append(req)

    def _paged_kv(self, tables: List[List[int]], ctx: List[int]) -> PagedKV:
        bm = self.block_manager
        width = max(len(t) for t in tables)
        rows = [t + [0] * (width - len(t)) for t in tables]  # padding past a row's keys is never read
        dev = bm.key_pool[0].device
        return PagedKV(bm.key_pool, bm.value_pool, torch.tensor(rows, dtype=torch.int32).to(dev),
                       torch.tensor(ctx, dtype=torch.int32).to(dev), max(ctx))

    @torch.no_grad()
    def _prefill(self, req: TTSRequest) -> torch.Tensor:
        """Prompt forward: its K/V go into the request's blocks; returns the first frame [K]."""
        kv = self._paged_kv([req.block_table], [req.seq_len])
        logits = self.model.decode_step_paged(req.prompt_codebooks.unsqueeze(0), kv)  # [1, K, V]
        return self._greedy(logits)[0]

    @torch.no_grad()
    def _decode(self, batch: List[TTSRequest]) -> torch.Tensor:
        """One frame for every request of the batch: [B, K] codebook tokens."""
        kv = self._paged_kv([r.block_table for r in batch], [r.seq_len + 1 for r in batch])
        inputs = torch.cat([r.last_frame_codebooks for r in batch], dim=0)  # [B, 1, K]
        return self._greedy(self.model.decode_step_paged(inputs, kv))

    def _greedy(self, logits: torch.Tensor) -> torch.Tensor:
        """Argmax per (request, codebook) row of logits [B, K, V] -> int64 [B, K]."""
        b, k, v = logits.shape
        return native.argmax(logits.reshape(b * k, v)).view(b, k)

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
        req.done = True
        self.block_manager.free_blocks(req.block_table)
        req.block_table = []
        self.completed.append(req)

    def _fail(self, req: TTSRequest, err: Exception) -> None:
        print(f"Error executing step for TTS request {req.id}: {err}")
        self._finish(req)
