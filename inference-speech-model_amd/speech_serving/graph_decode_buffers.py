"""Fixed decode slots replayed through captured HIP graphs.

Public interface of the reference's GraphDecodeBuffers
(speech_serving/graph_decode_buffers.py:124-638): constructor arguments,
assign_slot / release_slot / find_free_slot / active_slot_count /
capture_all_buckets / prepare_replay() -> bucket / replay_step(bucket) /
should_readback / sync_tokens / vram_overhead_mb, and the `slots`,
`g_cross_kv`, `cross_cache` (None), `_step_in_k` attributes.

Redesign for the paged pool:
  * Self-attention K/V lives in the BlockManager pool and is read through each
    slot's block table (uploaded once at assign_slot). There are no per-length
    bucket copies, no bucket upgrades and no self-KV zeroing.
  * Graphs are captured per BATCH bucket (BATCH_BUCKETS, capped at max_slots).
    Captured row r serves slot row_slot[r], so active slots need not be
    contiguous: a step uploads four int32 per row (slot, context length,
    encoder length, cross slot) from a pinned bank and replays the smallest
    bucket that holds every active slot. Idle rows point at a spare slot with
    zero lengths and do no work.
  * Each slot's next input token is kept on the device (g_slot_tokens); the
    captured argmax writes it back per slot, so a K-step readback window needs
    no token uploads.
  * Cross-attention reads g_cross_kv [S, L, 2, H, max_enc_len, D] (slot-major,
    filled once per request at assign_slot) with per-row valid lengths.
"""
from __future__ import annotations

import math
from typing import Any, Dict, List, Optional, Tuple

import torch

from . import native
from .block_manager import BlockManager
from .models import CrossKV, PagedKV

SELF_KV_BUCKETS = [64, 128, 256, 448]  # decoder length buckets of the reference (max decode length 448)
BATCH_BUCKETS = [1, 8, 16, 32, 64, 128]
MAX_SLOTS = 128
DEFAULT_READBACK_K = 1
MAX_BLOCKS = 64


def get_next_bucket(length: int) -> int:
    """Smallest decoder-length bucket >= length, or the largest (reference semantics)."""
    for b in SELF_KV_BUCKETS:
        if length <= b:
            return b
    return SELF_KV_BUCKETS[-1]


def batch_buckets(max_slots: int) -> List[int]:
    """Captured batch sizes: the standard buckets below max_slots, plus max_slots."""
    return sorted({b for b in BATCH_BUCKETS if b < max_slots} | {max_slots})


class SlotInfo:
    """Host-side state of one decode slot."""

    def __init__(self, slot_idx: int):
        self.slot_idx = slot_idx
        self.active = False
        self.req = None
        self.decoder_seq_len = 0
        self.last_token_id = 0
        self.generated_count = 0
        self.max_new_tokens = 0
        self.eos_token_id = None
        self.bucket = BATCH_BUCKETS[0]
        self.pending_tokens: List[int] = []
        self.eos_reached = False
        self.enc_seq_len = 0
        self.readback_start = 0
        self.needs_token_upload = False
        self.assignment_count = 0
        self.reused = False
        self.last_readback_trace: List[Dict[str, int]] = []
        self.block_table: List[int] = []


class GraphDecodeBuffers:
    def __init__(
        self,
        model: Any,
        device: str = "cuda",
        dtype: torch.dtype = torch.float16,
        max_slots: int = MAX_SLOTS,
        readback_k: int = DEFAULT_READBACK_K,
        max_blocks: int = MAX_BLOCKS,
        max_enc_len: int = 1500,
        non_blocking_copies: bool = True,
        zero_slot_buffers_on_release: bool = False,
        force_bucket: Optional[int] = None,
        block_manager: Optional[BlockManager] = None,
        capture: bool = True,
    ):
        if not callable(getattr(model, "decode_step_paged", None)):
            raise TypeError(
                f"GraphDecodeBuffers captures the model's paged decode step (decode_step_paged); "
                f"{type(model).__name__} exposes only decode_step, so serve it with graph_decode=False "
                "(the scheduler then runs it eagerly on K/V gathered from the pool)")
        self.model = model
        self.device = torch.device(device)
        self.dtype = dtype
        self.max_slots = int(max_slots)
        self.readback_k = max(int(readback_k), 1)
        self.max_blocks = int(max_blocks)
        self.max_enc_len = int(max_enc_len)
        self.non_blocking_copies = non_blocking_copies
        self.zero_slot_buffers_on_release = zero_slot_buffers_on_release
        self.buckets = batch_buckets(self.max_slots)
        if force_bucket is not None and force_bucket not in self.buckets:
            raise ValueError(f"force_bucket must be one of {self.buckets}, got {force_bucket}")
        self.force_bucket = force_bucket

        self.num_decoder_layers = model.num_decoder_layers
        self.num_encoder_layers = getattr(model, "num_encoder_layers", model.num_decoder_layers)
        self.num_heads = model.num_heads
        self.head_dim = model.head_dim
        self.hidden_dim = model.hidden_dim
        self.vocab_size = model.vocab_size

        if block_manager is None:
            block_manager = BlockManager(self.num_decoder_layers, self.num_heads, self.head_dim, 16,
                                         num_blocks=self.max_slots * self.max_blocks, dtype=dtype, device=str(device))
        if block_manager.dtype != dtype or block_manager.num_layers != self.num_decoder_layers:
            raise ValueError("block_manager dtype / layer count must match the graph buffers")
        self.bm = block_manager
        self.block_size = block_manager.block_size
        self.max_ctx = self.max_blocks * self.block_size

        S, dev = self.max_slots, self.device
        self.slots = [SlotInfo(i) for i in range(S)]
        self.cross_cache = None
        self.g_cross_kv = torch.zeros((S, self.num_decoder_layers, 2, self.num_heads, self.max_enc_len,
                                       self.head_dim), device=dev, dtype=dtype)
        # Row S of the tables / tokens is the spare slot idle rows point at.
        self.g_tables = torch.full((S + 1, self.max_blocks), -1, dtype=torch.int32, device=dev)
        self.g_slot_tokens = torch.zeros(S + 1, dtype=torch.int64, device=dev)
        # On-device EOS (the reference's g_finished state): per-slot EOS id (-1 = none) and finished flag. The
        # argmax of every step sets a slot's flag when it emits the slot's EOS id and counts it in
        # g_output_tokens[bmax], which travels to the host with the step's tokens.
        self.g_slot_eos = torch.full((S + 1,), -1, dtype=torch.int64, device=dev)
        self.g_slot_finished = torch.zeros(S + 1, dtype=torch.int32, device=dev)
        bmax = self.buckets[-1]
        self.g_rows = torch.zeros((4, bmax), dtype=torch.int32, device=dev)  # slot, ctx, enc_len, cross slot
        self.g_output_tokens = torch.zeros(bmax + 1, dtype=torch.int64, device=dev)  # tokens, then finished count

        # Two row banks: the host runs at most two steps ahead of the GPU, so a finished count that reaches
        # the host ring (see should_readback) is seen within about two steps whatever readback_k is.
        self._n_banks = 2
        self._banks = [torch.zeros((4, bmax), dtype=torch.int32).pin_memory() for _ in range(self._n_banks)]
        self._bank_events = [torch.cuda.Event() for _ in range(self._n_banks)]
        self._bank_in_flight = [False] * self._n_banks
        self.h_token_ring = torch.zeros((self.readback_k, bmax + 1), dtype=torch.int64).pin_memory()
        self._ring_events = [torch.cuda.Event() for _ in range(self.readback_k)]
        self._finished_seen = 0
        self.early_readbacks = 0
        self._readback_event = torch.cuda.Event()
        self._step_in_k = 0
        self._step_counter = 0
        self._window_buckets: List[int] = []
        self._window_rows: List[Dict[int, int]] = []

        self.graphs: Dict[int, torch.cuda.CUDAGraph] = {}
        self._graph_pool = None
        self._graph_workspace: Optional[torch.Tensor] = None
        if capture:
            self.capture_all_buckets()

    # ------------------------------------------------------------------ slots
    def find_free_slot(self) -> Optional[int]:
        for s in self.slots:
            if not s.active:
                return s.slot_idx
        return None

    def active_slot_count(self) -> int:
        return sum(1 for s in self.slots if s.active)

    def assign_slot(self, req: Any, enc_kv_layers: List[Tuple[torch.Tensor, torch.Tensor]], prompt_len: int,
                    initial_tok: int, initial_self_kv: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None) -> int:
        """Bind a request to a free slot: its block table, encoder K/V and first token.

        req.decoder_block_table must already cover prompt_len + max_new_tokens
        positions. If initial_self_kv ([1, H, P, D] per layer) is given it is
        written into the pool at positions 0..P-1 (the scheduler's prefill
        normally wrote them already; the bytes are the same).
        """
        slot_idx = self.find_free_slot()
        if slot_idx is None:
            raise RuntimeError("No free slot available in GraphDecodeBuffers!")
        table = list(req.decoder_block_table)
        if len(table) > self.max_blocks:
            raise RuntimeError(f"request needs {len(table)} blocks; slots hold at most {self.max_blocks}")
        s = self.slots[slot_idx]
        s.active = True
        s.req = req
        s.decoder_seq_len = prompt_len
        s.last_token_id = initial_tok
        s.generated_count = 1
        s.max_new_tokens = req.max_new_tokens
        s.eos_token_id = req.eos_token_id
        s.pending_tokens = [initial_tok]
        s.eos_reached = False
        s.enc_seq_len = min(enc_kv_layers[0][0].shape[2], self.max_enc_len) if enc_kv_layers else 0
        s.readback_start = self._step_in_k
        s.needs_token_upload = False
        s.reused = s.assignment_count > 0
        s.assignment_count += 1
        s.last_readback_trace = []
        s.block_table = table

        layers = enc_kv_layers[: self.num_decoder_layers]
        if layers:  # every layer's encoder K/V into the slot in one launch
            native.copy_cross_kv([ck[0] for ck, _ in layers], [cv[0] for _, cv in layers], self.g_cross_kv[slot_idx],
                                 min(layers[0][0].shape[2], self.max_enc_len))
        row = torch.full((self.max_blocks,), -1, dtype=torch.int32)
        row[: len(table)] = torch.tensor(table, dtype=torch.int32)
        self.g_tables[slot_idx].copy_(row.to(self.device))
        if initial_self_kv is not None:
            p = min(initial_self_kv[0][0].shape[2], prompt_len)
            slots = torch.tensor([self.bm.slot(table, i) for i in range(p)], dtype=torch.int64, device=self.device)
            for l, (sk, sv) in enumerate(initial_self_kv):
                native.append(sk[0, :, :p].transpose(0, 1), sv[0, :, :p].transpose(0, 1), self.bm.key_pool[l],
                              self.bm.value_pool[l], slots)
        self.g_slot_tokens[slot_idx].fill_(int(initial_tok))
        eos = getattr(req, "eos_token_id", None)
        self.g_slot_eos[slot_idx].fill_(int(eos) if eos is not None and eos >= 0 else -1)
        self.g_slot_finished[slot_idx].zero_()
        return slot_idx

    def set_first_token(self, slot_idx: int, tok: int) -> None:
        """Record the first token of a slot bound before its prefill ran (the scheduler binds the
        slots of a step's admissions, prefills them as one batch, then sets each first token)."""
        s = self.slots[slot_idx]
        s.last_token_id = tok
        s.pending_tokens = [tok]
        self.g_slot_tokens[slot_idx].fill_(int(tok))

    def release_slot(self, slot_idx: int) -> None:
        s = self.slots[slot_idx]
        s.active = False
        s.req = None
        s.pending_tokens = []
        s.eos_reached = False
        s.needs_token_upload = False
        s.readback_start = 0
        s.last_readback_trace = []
        s.block_table = []
        if self.zero_slot_buffers_on_release:
            self.g_cross_kv[slot_idx].zero_()
            self.g_tables[slot_idx].fill_(-1)

    # ------------------------------------------------------------------ capture
    def _forward_step(self, bucket: int) -> None:
        rows = self.g_rows[:, :bucket]
        row_slot, ctx, enc, cslot = rows[0], rows[1], rows[2], rows[3]
        ids = self.g_slot_tokens.index_select(0, row_slot).view(bucket, 1)
        # prepare_replay lays the rows out longest-first (idle rows, of length 0, last)
        kv = PagedKV(self.bm.key_pool, self.bm.value_pool, self.g_tables, ctx, self.max_ctx, table_rows=row_slot,
                     rows_longest_first=True)
        cross = CrossKV([self.g_cross_kv[:, l, 0] for l in range(self.num_decoder_layers)],
                        [self.g_cross_kv[:, l, 1] for l in range(self.num_decoder_layers)],
                        enc, self.max_enc_len, slot_ids=cslot)
        logits = self.model.decode_step_paged(ids, kv, cross)
        bmax = self.buckets[-1]
        native.argmax(logits, out=self.g_output_tokens[:bucket], row_slots=row_slot, slot_tokens=self.g_slot_tokens,
                      slot_eos=self.g_slot_eos, slot_finished=self.g_slot_finished,
                      finished_count=self.g_output_tokens[bmax:])

    def _idle_rows(self) -> None:
        idle = torch.zeros((4, self.g_rows.shape[1]), dtype=torch.int32)
        idle[0] = self.max_slots
        self.g_rows.copy_(idle.to(self.device))

    def capture_all_buckets(self, warmup_steps: int = 2) -> None:
        """Capture one graph per batch bucket, sharing one memory pool."""
        for b in self.buckets:
            native.reserve_attention(b, self.num_heads, self.head_dim, self.max_ctx, self.dtype, self.device)
            native.reserve_attention(b, self.num_heads, self.head_dim, self.max_enc_len, self.dtype, self.device)
        self._idle_rows()
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.no_grad():
            for b in self.buckets:
                with torch.cuda.stream(side):
                    for _ in range(warmup_steps):
                        self._forward_step(b)
                torch.cuda.current_stream(self.device).wait_stream(side)
                g = torch.cuda.CUDAGraph()
                kwargs = {"pool": self._graph_pool} if self._graph_pool is not None else {}
                with torch.cuda.graph(g, stream=side, **kwargs):
                    self._forward_step(b)
                if self._graph_pool is None:
                    self._graph_pool = g.pool()
                self.graphs[b] = g
        # The graphs hold the attention workspace's address: keep that buffer alive even if a
        # later, larger eager call grows the device's workspace (which drops the old one).
        self._graph_workspace = native.reserve_workspace(0, self.device)
        torch.cuda.synchronize(self.device)

    # ------------------------------------------------------------------ stepping
    def pick_bucket(self, n_active: int) -> int:
        if self.force_bucket is not None:
            if n_active > self.force_bucket:
                raise RuntimeError(f"{n_active} active slots exceed the forced bucket {self.force_bucket}")
            return self.force_bucket
        for b in self.buckets:
            if b >= n_active:
                return b
        return self.buckets[-1]

    def prepare_replay(self) -> int:
        """Fill a pinned bank with the active slots' rows and upload it; returns the bucket."""
        # Rows longest-first: the attention workgroups of a launch then land on the
        # compute units with long and short contexts mixed, which evens the
        # per-unit load. The row -> slot map of every step is kept for readback.
        active = sorted((s for s in self.slots if s.active), key=lambda s: -s.decoder_seq_len)
        bucket = self.pick_bucket(len(active))
        bank_idx = self._step_counter % self._n_banks
        if self._bank_in_flight[bank_idx]:
            self._bank_events[bank_idx].synchronize()
            self._bank_in_flight[bank_idx] = False
        bank = self._banks[bank_idx]
        bank[0].fill_(self.max_slots)
        bank[1:].zero_()
        rows: Dict[int, int] = {}
        for i, s in enumerate(active):
            pos = s.decoder_seq_len
            if pos + 1 > self.max_ctx or pos // self.block_size >= len(s.block_table):
                raise RuntimeError(f"slot {s.slot_idx}: position {pos} is outside its {len(s.block_table)} blocks")
            bank[0, i] = s.slot_idx
            bank[1, i] = pos + 1
            bank[2, i] = s.enc_seq_len
            bank[3, i] = s.slot_idx
            s.bucket = bucket
            rows[s.slot_idx] = i
        self._window_rows_pending = rows
        self.g_rows.copy_(bank, non_blocking=self.non_blocking_copies)
        if self.non_blocking_copies:
            self._bank_events[bank_idx].record()
            self._bank_in_flight[bank_idx] = True
        return bucket

    def replay_step(self, bucket: int) -> None:
        if bucket not in self.graphs:
            self.capture_all_buckets()
        self.graphs[bucket].replay()
        if self._step_in_k < self.h_token_ring.shape[0]:
            # Every row plus the finished count: one small copy per step, as before.
            self.h_token_ring[self._step_in_k].copy_(self.g_output_tokens, non_blocking=self.non_blocking_copies)
            self._ring_events[self._step_in_k].record()
            self._window_buckets.append(bucket)
            self._window_rows.append(getattr(self, "_window_rows_pending", {}))
            self._step_in_k += 1
        self._step_counter += 1
        for s in self.slots:
            if s.active:
                s.decoder_seq_len += 1
                s.generated_count += 1

    def should_readback(self) -> bool:
        if self._step_counter % self.readback_k == 0 or self._step_in_k >= self.h_token_ring.shape[0]:
            return True
        if any(s.active and s.generated_count >= s.max_new_tokens for s in self.slots):
            return True
        return self._eos_seen_on_device()

    def _eos_seen_on_device(self) -> bool:
        """True when the newest ring entry that has already landed (checked without waiting) counts more
        finished slots than the last readback saw: a request emitted EOS inside the window."""
        bmax = self.buckets[-1]
        for k in range(self._step_in_k - 1, -1, -1):
            if self._ring_events[k].query():
                if int(self.h_token_ring[k, bmax]) > self._finished_seen:
                    self.early_readbacks += 1
                    return True
                return False
        return False

    def sync_tokens(self) -> List[Tuple[SlotInfo, List[int]]]:
        """Wait for the window's replays and return each active slot's new tokens."""
        self._readback_event.record()
        self._readback_event.synchronize()
        self._bank_in_flight = [False] * self._n_banks
        ring = self.h_token_ring.tolist()
        if self._step_in_k:
            self._finished_seen = ring[self._step_in_k - 1][self.buckets[-1]]
        results = []
        for s in self.slots:
            if not s.active:
                continue
            toks, trace = [], []
            for k in range(s.readback_start, self._step_in_k):
                row = self._window_rows[k].get(s.slot_idx)
                if row is None:
                    continue
                toks.append(int(ring[k][row]))
                trace.append({"bucket": self._window_buckets[k], "readback_position": k})
            s.last_readback_trace = trace
            if toks:
                s.last_token_id = toks[-1]
                s.pending_tokens.extend(toks)
            results.append((s, toks))
            s.readback_start = 0
        self._step_in_k = 0
        self._window_buckets = []
        self._window_rows = []
        return results

    def vram_overhead_mb(self) -> float:
        """Device bytes held by the slot buffers (cross K/V, tables, tokens, row inputs)."""
        total = sum(t.numel() * t.element_size() for t in (self.g_cross_kv, self.g_tables, self.g_slot_tokens,
                                                            self.g_slot_eos, self.g_slot_finished, self.g_rows,
                                                            self.g_output_tokens))
        return total / (1024 * 1024)
