"""Phase-aware continuous-batching scheduler over the paged decoder pool.

Public interface of the reference's PhaseAwareSpeechScheduler
(speech_serving/phase_aware_scheduler.py:125-1243): constructor flags,
submit() with high-water-mark admission, step() / has_work() /
run_until_done(), the `queue` / `active_decode` / `completed` lists,
`graph_buffers`, DualCacheRequest fields, telemetry getters, and the EOS
conventions (eager keeps the EOS token as the last generated token; graph
decode trims EOS and everything after it, :739-766 vs the eager :1022-1036).

What changed for MI355X: the decoder pool is authoritative. Prefill and every
decode step append K/V into BlockManager blocks and attend through the block
tables in the same HIP launch, so there is no per-request contiguous working
KV, no per-step cat/zero-pad batching and no padding masks (:795-846 of the
reference). Cross-attention reads one slot-major encoder K/V arena with
per-row lengths (the reference's bool/additive masks, :884-887).
Attention over masked padding equals attention over the valid prefix, so the
token streams are those of the reference's eager path.
"""
from __future__ import annotations

import enum
import hashlib
import logging
import time
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

from . import native
from .dual_cache_manager import DualCacheManager
from .graph_decode_buffers import MAX_SLOTS, DEFAULT_READBACK_K, GraphDecodeBuffers
from .memory_guard import MemoryGuard, logger
from .models import KVCache, LayerKV, PagedKVCache
from .phase_timing import PhaseTimer

WHISPER_SOT_TOKEN_ID = 50258
WHISPER_LANG_EN_TOKEN_ID = 50259
WHISPER_TRANSCRIBE_TOKEN_ID = 50359
WHISPER_NO_TIMESTAMPS_TOKEN_ID = 50363
WHISPER_EOS_TOKEN_ID = 50257
WHISPER_DEFAULT_PREFIX_TOKENS = [WHISPER_SOT_TOKEN_ID, WHISPER_LANG_EN_TOKEN_ID, WHISPER_TRANSCRIBE_TOKEN_ID,
                                 WHISPER_NO_TIMESTAMPS_TOKEN_ID]


class RequestPhase(enum.Enum):
    QUEUED = "QUEUED"
    ENCODE_PHASE = "ENCODE_PHASE"
    DECODE_PHASE = "DECODE_PHASE"
    COMPLETED = "COMPLETED"
    FAILED = "FAILED"


@dataclass
class DualCacheRequest:
    id: int
    mel_features: torch.Tensor
    prompt_token_ids: torch.Tensor
    max_new_tokens: int
    arrival_time: float = 0.0
    eos_token_id: Optional[int] = None
    full_input_hash: Optional[str] = None
    phase: RequestPhase = RequestPhase.QUEUED
    encoder_seq_len: int = 0
    encoder_block_table: List[int] = field(default_factory=list)
    decoder_seq_len: int = 0
    decoder_block_table: List[int] = field(default_factory=list)
    generated_tokens: List[int] = field(default_factory=list)
    generated_count: int = 0
    last_token_id: Optional[int] = None
    done: bool = False
    slot_idx: Optional[int] = None
    graph_slot_idx: Optional[int] = None
    graph_slot_reused: bool = False
    graph_token_trace: List[Dict[str, int]] = field(default_factory=list)
    graph_extra_slot_steps: int = 0
    cached_encoder_kv: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None
    cached_decoder_kv: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None
    cross_slot: Optional[int] = None
    cross_layers: int = 0
    encoded_kv: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None
    submission_time: Optional[float] = None
    arrival_wall_time: Optional[float] = None
    queue_wait_time: Optional[float] = None
    start_time: Optional[float] = None
    encode_done_time: Optional[float] = None
    first_token_time: Optional[float] = None
    finish_time: Optional[float] = None
    phase_timing: Optional[Dict[str, Any]] = None


class CrossArena:
    """Slot-major encoder K/V for eager decode: [S, L, 2, H, T, D].

    The live requests hold slots 0..n-1: a released slot is refilled by moving the last live
    slot into it. A batch laid out in slot order therefore reads its encoder K/V as the
    per-layer views buf[lo:hi, l, 0|1, :, :T], the [B, H, T, D] tensors that decode_step
    takes as encoder_past_kv_list (the reference batches each step's encoder K/V into such
    tensors, phase_aware_scheduler.py:848-970). T grows (reallocate + copy of the live
    slots) when a request needs more encoder positions than the arena holds.
    """

    def __init__(self, slots: int, layers: int, heads: int, head_dim: int, dtype, device):
        self.slots, self.layers, self.heads, self.head_dim = slots, layers, heads, head_dim
        self.dtype, self.device = dtype, device
        self.buf: Optional[torch.Tensor] = None
        self.owner: List[Any] = []  # owner[s]: the request in slot s
        self.lens: List[int] = []  # encoder positions held in slot s

    @property
    def max_len(self) -> int:
        return 0 if self.buf is None else self.buf.shape[4]

    def _ensure(self, t: int) -> None:
        if self.buf is not None and t <= self.buf.shape[4]:
            return
        new_t = max(t, 1500 if self.buf is None else 2 * self.buf.shape[4])
        new = torch.zeros((self.slots, self.layers, 2, self.heads, new_t, self.head_dim), dtype=self.dtype,
                          device=self.device)
        if self.buf is not None:
            for s, n in enumerate(self.lens):
                new[s, :, :, :, :n].copy_(self.buf[s, :, :, :, :n])
        self.buf = new

    def _take(self, req, t: int) -> int:
        if len(self.owner) >= self.slots:
            raise RuntimeError("cross-attention arena is full")
        self._ensure(t)
        s = len(self.owner)
        self.owner.append(req)
        self.lens.append(t)
        req.cross_slot = s
        return s

    def put(self, req, enc_kv: List[Tuple[torch.Tensor, torch.Tensor]]) -> int:
        """Copy one request's per-layer K/V [1, H, T, D] into the next slot; returns the slot."""
        t = enc_kv[0][0].shape[2]
        s = self._take(req, t)
        for l, (k, v) in enumerate(enc_kv[: self.layers]):
            self.buf[s, l, 0, :, :t].copy_(k[0])
            self.buf[s, l, 1, :, :t].copy_(v[0])
        return s

    def put_from_pool(self, req, enc_bm, block_table: List[int], t: int, layers: int) -> int:
        """Gather a request's encoder K/V from the encoder pool straight into the next slot."""
        s = self._take(req, t)
        dev = self.buf.device
        tbl = torch.tensor([block_table], dtype=torch.int32, device=dev)
        lens = torch.tensor([t], dtype=torch.int32, device=dev)
        tmax = self.buf.shape[4]
        for l in range(min(layers, self.layers)):
            native.gather(enc_bm.key_pool[l], enc_bm.value_pool[l], tbl, lens, tmax,
                          k_out=self.buf[s, l, 0].unsqueeze(0), v_out=self.buf[s, l, 1].unsqueeze(0))
        return s

    def release(self, req) -> None:
        s = getattr(req, "cross_slot", None)
        if s is None or s >= len(self.owner) or self.owner[s] is not req:
            return
        last = len(self.owner) - 1
        if s != last:
            n = self.lens[last]
            self.buf[s, :, :, :, :n].copy_(self.buf[last, :, :, :, :n])
            self.owner[s], self.lens[s] = self.owner[last], n
            self.owner[s].cross_slot = s
        self.owner.pop()
        self.lens.pop()
        req.cross_slot = None

    def views(self, lo: int, hi: int, t: int, layers: int) -> List[Tuple[torch.Tensor, torch.Tensor]]:
        """Per-layer (K, V) [hi - lo, H, t, D] of slots lo..hi-1."""
        return [(self.buf[lo:hi, l, 0, :, :t], self.buf[lo:hi, l, 1, :, :t]) for l in range(layers)]


def _slot_runs(reqs: List["DualCacheRequest"], slot_of) -> List[List["DualCacheRequest"]]:
    """reqs in slot order, cut where the slots stop being consecutive."""
    runs: List[List[DualCacheRequest]] = []
    for r in sorted(reqs, key=slot_of):
        if runs and slot_of(r) == slot_of(runs[-1][-1]) + 1:
            runs[-1].append(r)
        else:
            runs.append([r])
    return runs


class PhaseAwareSpeechScheduler:
    def __init__(
        self,
        model,
        dual_cache_manager: DualCacheManager,
        memory_guard: Optional[MemoryGuard] = None,
        max_batch_size: int = 32,
        retain_encoder_cache: bool = False,
        step_delay: float = 0.0,
        verbose: bool = False,
        device: str = "cuda",
        eos_token_id: Optional[int] = None,
        max_cached_encoder_inputs: int = 100,
        cache_cross_kv: bool = False,
        batch_encoder: bool = False,
        no_sync_decode: bool = False,
        avoid_redundant_cross_kv: bool = False,
        graph_decode: bool = False,
        graph_readback_k: int = DEFAULT_READBACK_K,
        graph_non_blocking_copies: bool = True,
        graph_zero_slot_buffers_on_release: bool = False,
        graph_force_bucket: Optional[int] = None,
        graph_direct_encoder_kv: bool = False,
        phase_timing: bool = False,
        graph_max_enc_len: int = 1500,
        graph_max_blocks: int = 64,
    ):
        self.model = model
        # Models with the paged step take a PagedKVCache as decode_step's past_key_values; a model
        # that exposes only the reference's decode_step is served on gathered contiguous K/V.
        self._paged_model = callable(getattr(model, "decode_step_paged", None))
        self.dual_cache = dual_cache_manager
        self.memory_guard = memory_guard or MemoryGuard()
        self.max_batch_size = max_batch_size
        self.retain_encoder_cache = retain_encoder_cache
        self.step_delay = step_delay
        self.verbose = verbose
        self.device = device
        self.eos_token_id = eos_token_id
        self.max_cached_encoder_inputs = max_cached_encoder_inputs
        # cache_cross_kv / avoid_redundant_cross_kv / no_sync_decode select among the
        # reference's cross-KV and sampling variants; here cross K/V is copied
        # once into the arena and sampling is one batched argmax, for every value.
        self.cache_cross_kv = cache_cross_kv
        self.batch_encoder = batch_encoder
        self.no_sync_decode = no_sync_decode
        self.avoid_redundant_cross_kv = avoid_redundant_cross_kv
        self.graph_decode = graph_decode
        self.graph_readback_k = graph_readback_k
        self.graph_direct_encoder_kv = bool(graph_direct_encoder_kv)
        if self.graph_direct_encoder_kv and (not self.graph_decode or self.retain_encoder_cache):
            raise ValueError("graph_direct_encoder_kv requires graph_decode=True and retain_encoder_cache=False")
        self.phase_timing = bool(phase_timing)
        self.phase_timer = PhaseTimer(self.phase_timing, device=self.device)
        dec_bm = self.dual_cache.decoder_bm
        self.graph_buffers: Optional[GraphDecodeBuffers] = None
        if self.graph_decode:
            self.max_batch_size = min(self.max_batch_size, MAX_SLOTS)
            self.graph_buffers = GraphDecodeBuffers(
                model=self.model, device=self.device, dtype=dec_bm.dtype, max_slots=self.max_batch_size,
                readback_k=self.graph_readback_k, max_blocks=graph_max_blocks, max_enc_len=graph_max_enc_len,
                non_blocking_copies=graph_non_blocking_copies,
                zero_slot_buffers_on_release=graph_zero_slot_buffers_on_release,
                force_bucket=graph_force_bucket, block_manager=dec_bm)
        self.cross_arena: Optional[CrossArena] = None
        if not self.graph_decode:
            self.cross_arena = CrossArena(self.max_batch_size, model.num_decoder_layers, model.num_heads,
                                          model.head_dim, dec_bm.dtype, torch.device(device))

        self.queue: List[DualCacheRequest] = []
        self.active_encode: List[DualCacheRequest] = []
        self.active_decode: List[DualCacheRequest] = []
        self.completed: List[DualCacheRequest] = []
        self._next_id = 0
        self.peak_in_flight_requests = 0
        self.peak_actually_used_bytes = 0
        self.peak_pool_blocks_used_bytes = 0
        self.rejected_requests_count = 0
        self.in_flight_history: List[int] = []
        self.queue_wait_times: List[float] = []
        self.retained_encoder_caches: Dict[int, Tuple[List[int], float]] = {}
        self.encoder_calls = 0
        self.encoder_calls_skipped = 0
        self.encode_time_saved_s = 0.0
        self._full_input_enc_cache: Dict[str, Dict[str, Any]] = {}
        self.decode_steps = 0
        self.decode_time_s = 0.0

    # ------------------------------------------------------------------ admission
    def submit(self, mel_features: torch.Tensor, prompt_token_ids: Optional[torch.Tensor] = None,
               max_new_tokens: int = 50, arrival_time: float = 0.0, eos_token_id: Optional[int] = None,
               arrival_wall_time: Optional[float] = None,
               _encoded_kv: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None) -> Optional[int]:
        """Queue a request; returns its id, or None when admission would cross the high-water mark."""
        enc_bm, dec_bm = self.dual_cache.encoder_bm, self.dual_cache.decoder_bm
        mel_in = mel_features.unsqueeze(0) if mel_features.dim() == 2 else mel_features
        encoded = _encoded_kv is not None
        full_hash = self._compute_full_input_hash(mel_in) if (self.retain_encoder_cache and not encoded) else None
        is_hit = bool(full_hash and full_hash in self._full_input_enc_cache)
        mel_len = mel_features.shape[-1]
        enc_len = (mel_len + 1) // 2
        direct = self.graph_direct_encoder_kv
        req_enc = 0 if (is_hit or direct or encoded) else -(-enc_len // enc_bm.block_size)
        req_dec = -(-max_new_tokens // dec_bm.block_size)
        q_enc = 0 if direct else sum(
            0 if (r.encoded_kv is not None
                  or (self.retain_encoder_cache and r.full_input_hash in self._full_input_enc_cache))
            else -(-((r.mel_features.shape[-1] + 1) // 2) // enc_bm.block_size) for r in self.queue)
        q_dec = sum(-(-r.max_new_tokens // dec_bm.block_size) for r in self.queue)

        def projected():
            es, ds = enc_bm.get_stats(), dec_bm.get_stats()
            pe = (es["allocated_blocks"] + q_enc + req_enc) / es["num_blocks"] * 100.0 if es["num_blocks"] else 0.0
            pd = (ds["allocated_blocks"] + q_dec + req_dec) / ds["num_blocks"] * 100.0 if ds["num_blocks"] else 0.0
            return pe, pd

        hwm = self.memory_guard.high_water_mark_pct
        pe, pd = projected()
        if pe >= hwm or pd >= hwm:
            freed = self._evict_retained_encoder_caches()
            if freed > 0:
                self.memory_guard.trigger_bulk_eviction_cleanup(freed, reason="high_water_mark_eviction")
            pe, pd = projected()
            if pe >= hwm or pd >= hwm:
                logger.warning(f"request refused: admitting it would fill the KV pools to {max(pe, pd):.1f}% "
                               f"(limit {hwm}%)")
                self.rejected_requests_count += 1
                return None

        if prompt_token_ids is None:
            if getattr(self.model, "vocab_size", 0) >= 50364:
                prompt_token_ids = torch.tensor([WHISPER_DEFAULT_PREFIX_TOKENS], dtype=torch.long)
            else:
                prompt_token_ids = torch.tensor([[1]], dtype=torch.long)
        eos = eos_token_id if eos_token_id is not None else self.eos_token_id
        if eos is None and getattr(self.model, "vocab_size", 0) >= 50258:
            eos = WHISPER_EOS_TOKEN_ID
        now = time.perf_counter()
        req = DualCacheRequest(id=self._next_id, mel_features=mel_features.to(self.device),
                               prompt_token_ids=prompt_token_ids.to(self.device), max_new_tokens=max_new_tokens,
                               arrival_time=arrival_time,
                               arrival_wall_time=arrival_wall_time if arrival_wall_time is not None else now,
                               submission_time=now, eos_token_id=eos, full_input_hash=full_hash,
                               encoded_kv=_encoded_kv)
        self._next_id += 1
        self.queue.append(req)
        return req.id

    def submit_encoded(self, encoder_kv: List[Tuple[torch.Tensor, torch.Tensor]],
                       prompt_token_ids: Optional[torch.Tensor] = None, max_new_tokens: int = 50,
                       arrival_time: float = 0.0, eos_token_id: Optional[int] = None,
                       arrival_wall_time: Optional[float] = None) -> Optional[int]:
        """Queue a request whose encoder output is already computed: one (K, V)
        [1, H, T_enc, D] pair per decoder layer (e.g. from model.project_cross_kv).
        The encode phase hands it straight to prefill; admission counts its
        T_enc positions like a mel input of 2*T_enc frames."""
        t_enc = encoder_kv[0][0].shape[2]
        placeholder = torch.empty((1, 2 * t_enc - 1), device="cpu")
        return self.submit(placeholder, prompt_token_ids, max_new_tokens, arrival_time, eos_token_id,
                           arrival_wall_time, _encoded_kv=encoder_kv)

    def _compute_full_input_hash(self, mel_in: torch.Tensor) -> str:
        """md5 of the full mel input (fp32 bytes) plus its dtype (reference :360-383)."""
        flat = mel_in.detach().cpu().to(torch.float32).numpy().tobytes()
        return hashlib.md5(flat + str(mel_in.dtype).encode()).hexdigest()

    def _evict_retained_encoder_caches(self, min_blocks_to_free: int = 1) -> int:
        freed = 0
        for h in sorted(self._full_input_enc_cache, key=lambda k: self._full_input_enc_cache[k]["last_access_time"]):
            entry = self._full_input_enc_cache.pop(h)
            if entry.get("held_by_cache"):
                freed += self.dual_cache.encoder_bm.release_blocks(entry["block_table"])
            if min_blocks_to_free > 0 and freed >= min_blocks_to_free:
                break
        return freed

    def flush_retained_caches(self) -> int:
        freed = self._evict_retained_encoder_caches(min_blocks_to_free=0)
        if freed > 0:
            self.memory_guard.trigger_bulk_eviction_cleanup(freed, reason="flush_retained_caches")
        return freed

    def flush_full_input_cache(self) -> int:
        n = len(self._full_input_enc_cache)
        for entry in self._full_input_enc_cache.values():
            if entry.get("held_by_cache"):
                self.dual_cache.encoder_bm.release_blocks(entry["block_table"])
        self._full_input_enc_cache.clear()
        return n

    # ------------------------------------------------------------------ encode
    def _admission_slots(self) -> int:
        return self.max_batch_size - (len(self.active_encode) + len(self.active_decode))

    def _process_encode_phase(self) -> None:
        enc_bm = self.dual_cache.encoder_bm
        placed = len(self.active_encode)
        while self._admission_slots() > 0 and self.queue:
            req = self.queue[0]
            mel_in = req.mel_features.unsqueeze(0) if req.mel_features.dim() == 2 else req.mel_features
            enc_len = (mel_in.shape[-1] + 1) // 2
            if req.full_input_hash is None and req.encoded_kv is None:
                req.full_input_hash = self._compute_full_input_hash(mel_in)
            hit = (self.retain_encoder_cache and req.encoded_kv is None
                   and req.full_input_hash in self._full_input_enc_cache)
            need = 0 if (hit or self.graph_direct_encoder_kv or req.encoded_kv is not None) \
                else -(-enc_len // enc_bm.block_size)
            if enc_bm.num_free_blocks < need:
                freed = self._evict_retained_encoder_caches()
                if freed > 0:
                    self.memory_guard.trigger_bulk_eviction_cleanup(freed, reason="encode_phase_capacity")
                if enc_bm.num_free_blocks < need:
                    break
            if self.graph_decode and self.graph_buffers.find_free_slot() is None:
                break
            self.queue.pop(0)
            req.start_time = time.perf_counter()
            ref = req.arrival_wall_time if req.arrival_wall_time is not None else req.submission_time
            if ref is not None:
                req.queue_wait_time = req.start_time - ref
                self.queue_wait_times.append(req.queue_wait_time)
            req.phase = RequestPhase.ENCODE_PHASE
            try:
                if hit:
                    entry = self._full_input_enc_cache[req.full_input_hash]
                    entry["last_access_time"] = time.perf_counter()
                    for blk in entry["block_table"]:
                        enc_bm.ref_counts[blk] += 1
                        enc_bm.total_lookups += 1
                        enc_bm.cache_hits += 1
                    req.encoder_block_table = list(entry["block_table"])
                    self.encoder_calls_skipped += 1
                    self.encode_time_saved_s += entry.get("encode_time", 0.0)
                    self._setup_request_after_encode(req, None, entry["cached_enc_kv"], full_hash=None,
                                                     enc_time=0.0, enc_seq_len=entry["enc_seq_len"])
                elif req.encoded_kv is not None:
                    kv, req.encoded_kv = req.encoded_kv, None
                    self._setup_request_after_encode(req, None, kv, full_hash=None, enc_seq_len=kv[0][0].shape[2],
                                                     use_encoder_pool=False)
                else:
                    t0 = time.perf_counter()
                    with torch.no_grad():
                        hidden, kv_list = self.model.encode(mel_in)
                    self.encoder_calls += 1
                    self._setup_request_after_encode(req, hidden, kv_list, full_hash=req.full_input_hash,
                                                     enc_time=time.perf_counter() - t0)
            except Exception as e:  # deterministic cleanup, reference :558-560
                logger.error(f"request {req.id} failed while encoding: {e}", exc_info=True)
                if req in self.active_encode:
                    self.active_encode.remove(req)
                self._complete_request(req, status=RequestPhase.FAILED)
        if len(self.active_encode) > placed:
            self._prefill_admitted(self.active_encode[placed:])

    def _setup_request_after_encode(self, req: DualCacheRequest, encoder_hidden: Optional[torch.Tensor],
                                    encoder_kv_list: List[Tuple[torch.Tensor, torch.Tensor]],
                                    full_hash: Optional[str] = None, enc_time: float = 0.0,
                                    enc_seq_len: Optional[int] = None, use_encoder_pool: bool = True) -> None:
        """Place the encoder K/V, allocate the decoder blocks and (graph decode) bind a slot. The prompt
        prefill and the first token follow in _prefill_admitted, batched over the step's admissions."""
        enc_bm, dec_bm = self.dual_cache.encoder_bm, self.dual_cache.decoder_bm
        t_enc = enc_seq_len if enc_seq_len is not None else encoder_hidden.shape[1]
        req.encoder_seq_len = t_enc
        direct = self.graph_direct_encoder_kv or not use_encoder_pool
        if not direct and not req.encoder_block_table:
            # Encoder pool is the source of truth (reference :578-606): write each layer's K/V into fresh blocks.
            table = [enc_bm.allocate_block(content_hash=None)[0] for _ in range(-(-t_enc // enc_bm.block_size))]
            req.encoder_block_table = table
            slots = torch.tensor([table[i // enc_bm.block_size] * enc_bm.block_size + i % enc_bm.block_size
                                  for i in range(t_enc)], dtype=torch.int64, device=self.device)
            for l, (k, v) in enumerate(encoder_kv_list[: enc_bm.num_layers]):
                native.append(k[0].transpose(0, 1), v[0].transpose(0, 1), enc_bm.key_pool[l], enc_bm.value_pool[l],
                              slots)
            if self.retain_encoder_cache and full_hash:
                for blk in table:
                    enc_bm.ref_counts[blk] += 1
                while len(self._full_input_enc_cache) >= self.max_cached_encoder_inputs:
                    oldest = min(self._full_input_enc_cache,
                                 key=lambda h: self._full_input_enc_cache[h]["last_access_time"])
                    entry = self._full_input_enc_cache.pop(oldest)
                    if entry.get("held_by_cache"):
                        enc_bm.release_blocks(entry["block_table"])
                self._full_input_enc_cache[full_hash] = {
                    "block_table": list(table), "enc_seq_len": t_enc, "cached_enc_kv": encoder_kv_list,
                    "last_access_time": time.perf_counter(), "held_by_cache": True, "encode_time": enc_time}
        req.cached_encoder_kv = encoder_kv_list
        req.cross_layers = min(len(encoder_kv_list), self.model.num_decoder_layers)
        req.encode_done_time = time.perf_counter()
        req.phase = RequestPhase.DECODE_PHASE

        p = req.prompt_token_ids.shape[-1]
        req.decoder_seq_len = p
        total = p + req.max_new_tokens if self.graph_decode else p
        for _ in range(-(-total // dec_bm.block_size)):
            req.decoder_block_table.append(self.dual_cache.allocate_decoder_block())

        # Cross-attention K/V for the prefill and the decode: the request's graph slot (filled by
        # assign_slot) or its arena slot (eager decode).
        if self.graph_decode:
            slot = self.graph_buffers.assign_slot(req=req, enc_kv_layers=encoder_kv_list, prompt_len=p,
                                                  initial_tok=0, initial_self_kv=None)
            req.slot_idx = slot
            req.graph_slot_idx = slot
            req.graph_slot_reused = self.graph_buffers.slots[slot].reused
        else:
            if req.encoder_block_table:
                self.cross_arena.put_from_pool(req, enc_bm, req.encoder_block_table, t_enc,
                                               min(self.model.num_decoder_layers, enc_bm.num_layers))
            else:
                self.cross_arena.put(req, encoder_kv_list)
        self.active_encode.append(req)

    def _prefill_admitted(self, reqs: List[DualCacheRequest]) -> None:
        """Prefill the prompts of the requests placed in this step and emit their first tokens.

        The reference prefills each request alone through model.decode_step and reads its first
        token back with .item() (phase_aware_scheduler.py:664-703). Here the requests that share a
        prompt length and a cross-attention layer count, and whose encoder K/V sit in consecutive
        slots, run as one batch: one model.decode_step over B x P prompt tokens (with a
        PagedKVCache, the K/V go into each request's blocks in the attention launch) and one token
        readback per batch. A batch that fails fails its requests, like a failed decode step. First
        tokens are then emitted in admission order."""
        groups: Dict[Tuple[int, int, bool], List[DualCacheRequest]] = {}
        for r in reqs:
            # A graph slot holds at most max_enc_len encoder positions; a longer encoder output
            # prefills from its own tensors (one request per launch).
            direct = self.graph_decode and r.encoder_seq_len > self.graph_buffers.max_enc_len
            groups.setdefault((r.prompt_token_ids.shape[-1], r.cross_layers, direct), []).append(r)
        first: Dict[int, int] = {}
        for (p, layers, direct), rs in groups.items():
            for part in ([[r] for r in rs] if direct else [rs]):
                try:
                    toks = self._prefill(part, p, layers, direct)
                except Exception as e:
                    logger.error(f"batched prefill of requests {[r.id for r in part]} failed: {e}", exc_info=True)
                    for r in part:
                        self.active_encode.remove(r)
                        self._complete_request(r, status=RequestPhase.FAILED)
                    continue
                first.update((id(r), t) for r, t in zip(part, toks))
        now = time.perf_counter()
        for req in reqs:
            if id(req) not in first:
                continue
            tok = first[id(req)]
            self.active_encode.remove(req)
            req.last_token_id = tok
            req.generated_tokens.append(tok)
            req.generated_count += 1
            req.first_token_time = now
            if (req.eos_token_id is not None and tok == req.eos_token_id) or req.generated_count >= req.max_new_tokens:
                self._complete_request(req, status=RequestPhase.COMPLETED)
                continue
            self.active_decode.append(req)
            if self.graph_decode:
                self.graph_buffers.set_first_token(req.slot_idx, tok)
            if self.avoid_redundant_cross_kv:
                req.cached_encoder_kv = None

    def _prefill(self, reqs: List[DualCacheRequest], p: int, layers: int, direct: bool) -> List[int]:
        """Prefill len(reqs) prompts of p tokens; returns each request's first token (in the order of reqs).
        One decode_step per run of requests whose encoder K/V occupy consecutive slots."""
        if direct:
            runs = [[r] for r in reqs]
        elif self.graph_decode:
            runs = _slot_runs(reqs, lambda r: r.slot_idx)
        else:
            runs = _slot_runs(reqs, lambda r: r.cross_slot)
        first: Dict[int, int] = {}
        for run in runs:
            first.update(zip(map(id, run), self._prefill_run(run, p, layers, direct)))
        return [first[id(r)] for r in reqs]

    def _encoder_inputs(self, run: List[DualCacheRequest], layers: int, direct: bool):
        """The run's encoder K/V as decode_step takes them: per layer (K, V) [n, H, T, D] (views of the
        slots), and the per-row lengths."""
        n = len(run)
        if direct:  # one request whose encoder output is longer than a graph slot: its own tensors
            kv = run[0].cached_encoder_kv[:layers]
            return [(k, v) for k, v in kv], [kv[0][0].shape[2]]
        if self.graph_decode:
            gb = self.graph_buffers
            lens = [min(r.encoder_seq_len, gb.max_enc_len) for r in run]
            t, lo = max(lens), run[0].slot_idx
            return [(gb.g_cross_kv[lo:lo + n, l, 0, :, :t], gb.g_cross_kv[lo:lo + n, l, 1, :, :t])
                    for l in range(layers)], lens
        lens = [r.encoder_seq_len for r in run]
        return self.cross_arena.views(run[0].cross_slot, run[0].cross_slot + n, max(lens), layers), lens

    @staticmethod
    def _encoder_mask(lens: List[int], lens_dev: torch.Tensor) -> Optional[torch.Tensor]:
        """The reference's bool encoder mask [n, 1, 1, T] when the rows' encoder lengths differ
        (phase_aware_scheduler.py:884-887), else None."""
        if min(lens) == max(lens):
            return None
        t = max(lens)
        return (torch.arange(t, device=lens_dev.device)[None, :] < lens_dev[:, None]).view(len(lens), 1, 1, t)

    def _prefill_run(self, run: List[DualCacheRequest], p: int, layers: int, direct: bool) -> List[int]:
        dec_bm = self.dual_cache.decoder_bm
        n = len(run)
        prompts = torch.cat([r.prompt_token_ids.reshape(1, p) for r in run]).to(self.device)
        enc_list, enc_lens = self._encoder_inputs(run, layers, direct)
        width = max(len(r.decoder_block_table) for r in run)
        meta = torch.full((n * width + 2 * n,), -1, dtype=torch.int32)  # tables [n, width], lengths, encoder lengths
        for i, r in enumerate(run):
            meta[i * width: i * width + len(r.decoder_block_table)] = torch.tensor(r.decoder_block_table,
                                                                                   dtype=torch.int32)
        meta[n * width: n * width + n] = p
        meta[n * width + n:] = torch.tensor(enc_lens, dtype=torch.int32)
        meta = meta.to(self.device)
        enc_dev = meta[n * width + n:]
        enc_mask = self._encoder_mask(enc_lens, enc_dev)
        with torch.no_grad():
            if self._paged_model:
                cache = PagedKVCache(dec_bm.key_pool, dec_bm.value_pool, meta[: n * width].view(n, width),
                                     meta[n * width: n * width + n], p, cross_lens=enc_dev, cross_mask=enc_mask)
                out = self.model.decode_step(input_ids=prompts, past_key_values=cache, encoder_past_kv_list=enc_list,
                                             encoder_attention_mask=enc_mask, use_cache=True, logits_to_keep=1)
            else:
                out = self.model.decode_step(input_ids=prompts, encoder_past_kv_list=enc_list,
                                             encoder_attention_mask=enc_mask, use_cache=True)
                self._append_prompt_kv(out.past_key_values, run, p)
            return native.argmax(out.logits[:, -1, :]).tolist()

    def _append_prompt_kv(self, cache, run: List[DualCacheRequest], p: int) -> None:
        """Write the prompt K/V a contiguous-cache model returned ([n, H, P, D] per layer) into each
        request's blocks, one skv_append per layer (the reference's block copies, :672-690)."""
        dec_bm = self.dual_cache.decoder_bm
        slots = torch.tensor([dec_bm.slot(r.decoder_block_table, i) for r in run for i in range(p)],
                             dtype=torch.int64).to(self.device)
        for l in range(dec_bm.num_layers):
            k, v = cache.layers[l].keys, cache.layers[l].values
            rows = k.shape[0] * p
            native.append(k[:, :, -p:].permute(0, 2, 1, 3).reshape(rows, k.shape[1], k.shape[3]),
                          v[:, :, -p:].permute(0, 2, 1, 3).reshape(rows, v.shape[1], v.shape[3]),
                          dec_bm.key_pool[l], dec_bm.value_pool[l], slots)

    # ------------------------------------------------------------------ decode
    def _staging(self, n: int) -> torch.Tensor:
        """Reusable pinned int32 buffer for one step's metadata upload. Each eager
        step ends with a device sync (token readback), so the previous upload
        from it has completed before it is refilled."""
        buf = getattr(self, "_staging_buf", None)
        if buf is None or buf.numel() < n:
            buf = torch.empty(max(n, 4096), dtype=torch.int32).pin_memory()
            self._staging_buf = buf
        return buf

    def _process_decode_phase(self) -> None:
        if not self.active_decode:
            return
        if self.graph_decode:
            self._process_decode_phase_graph()
            return
        t0 = time.perf_counter()
        dec_bm = self.dual_cache.decoder_bm
        bs = dec_bm.block_size
        # Block-boundary allocation (reference :780-783), one request at a time: a request
        # that cannot get its next block fails alone and leaves the batch; the others decode.
        starved = []
        for r in self.active_decode:
            if r.decoder_seq_len % bs == 0:
                try:
                    r.decoder_block_table.append(self.dual_cache.allocate_decoder_block())
                except RuntimeError as e:
                    logger.error(f"request {r.id}: no decoder block for position {r.decoder_seq_len}: {e}")
                    starved.append(r)
        for r in starved:
            self._complete_request(r, status=RequestPhase.FAILED)
        if starved:
            self.active_decode = [r for r in self.active_decode if r not in starved]
        if not self.active_decode:
            return
        tok_of: Dict[int, int] = {}
        try:
            # The batch in arena order: row b's encoder K/V is slot lo + b (one run when, as usual,
            # the active requests hold slots 0..B-1).
            for run in _slot_runs(self.active_decode, lambda r: r.cross_slot):
                tok_of.update(zip(map(id, run), self._decode_run(run)))
        except Exception as e:  # the batched step failed: release every request deterministically
            logger.error(f"batched decode step failed, releasing its requests: {e}", exc_info=True)
            for r in list(self.active_decode):
                self._complete_request(r, status=RequestPhase.FAILED)
            self.active_decode = []
            return
        still = []
        for r in self.active_decode:
            tok = tok_of[id(r)]
            r.decoder_seq_len += 1
            r.last_token_id = tok
            r.generated_tokens.append(tok)
            r.generated_count += 1
            if (r.eos_token_id is not None and tok == r.eos_token_id) or r.generated_count >= r.max_new_tokens:
                self._complete_request(r, status=RequestPhase.COMPLETED)
            else:
                still.append(r)
        self.active_decode = still
        self.decode_steps += 1
        self.decode_time_s += time.perf_counter() - t0

    def _decode_run(self, run: List[DualCacheRequest]) -> List[int]:
        """One decode step of the requests of run (encoder K/V in consecutive arena slots) through
        model.decode_step, as the reference's eager step (phase_aware_scheduler.py:982-991); returns
        each request's greedy token."""
        dec_bm = self.dual_cache.decoder_bm
        b = len(run)
        layers = run[0].cross_layers
        if any(r.cross_layers != layers for r in run):
            raise RuntimeError("requests in one decode batch must have encoder K/V for the same layers")
        maxblk = max(len(r.decoder_block_table) for r in run)
        staging = self._staging(b * (maxblk + 4))
        meta = staging.numpy()[: b * (maxblk + 4)].reshape(b, maxblk + 4)
        meta.fill(-1)
        for i, r in enumerate(run):
            meta[i, :len(r.decoder_block_table)] = r.decoder_block_table
            meta[i, maxblk] = r.decoder_seq_len + 1
            meta[i, maxblk + 1] = r.encoder_seq_len
            meta[i, maxblk + 2] = r.decoder_seq_len
            meta[i, maxblk + 3] = r.last_token_id
        dev = staging[: b * (maxblk + 4)].view(b, maxblk + 4).to(self.device, non_blocking=True)
        tables = dev[:, :maxblk].contiguous()
        ctx = dev[:, maxblk].contiguous()
        enc = dev[:, maxblk + 1].contiguous()
        pos = dev[:, maxblk + 2: maxblk + 3].to(torch.int64)
        ids = dev[:, maxblk + 3: maxblk + 4].to(torch.int64)
        enc_lens = [r.encoder_seq_len for r in run]
        enc_list = self.cross_arena.views(run[0].cross_slot, run[0].cross_slot + b, max(enc_lens), layers)
        enc_mask = self._encoder_mask(enc_lens, enc)
        with torch.no_grad():
            if self._paged_model:
                lens = meta[:, maxblk]
                cache = PagedKVCache(dec_bm.key_pool, dec_bm.value_pool, tables, ctx, int(lens.max()),
                                     cross_lens=enc, cross_mask=enc_mask,
                                     rows_longest_first=bool((lens[1:] <= lens[:-1]).all()))
                out = self.model.decode_step(input_ids=ids, past_key_values=cache, encoder_past_kv_list=enc_list,
                                             attention_mask=None, encoder_attention_mask=enc_mask, position_ids=pos,
                                             use_cache=True, logits_to_keep=1)
            else:
                out = self._decode_run_contiguous(run, tables, ctx, ids, pos, enc_list, enc_mask)
            return native.argmax(out.logits[:, -1, :]).tolist()

    def _decode_run_contiguous(self, run, tables, ctx, ids, pos, enc_list, enc_mask):
        """A model with only the reference's decode_step: each row's past K/V is gathered from the pool
        into a zero-padded [B, H, T, D] batch (skv_gather) with the reference's padding mask
        (:818-846), the model steps, and the new token's K/V goes back into the pool (skv_append)
        from the returned cache (:1001-1010)."""
        dec_bm = self.dual_cache.decoder_bm
        seq = [r.decoder_seq_len for r in run]
        tmax = max(seq)
        past = ctx - 1
        cache = KVCache([LayerKV(*native.gather(dec_bm.key_pool[l], dec_bm.value_pool[l], tables, past, tmax))
                         for l in range(dec_bm.num_layers)])
        mask = None
        if len(run) > 1 and min(seq) < tmax:
            m = torch.ones((len(run), tmax + 1), dtype=torch.long)
            for i, n in enumerate(seq):
                m[i, n:tmax] = 0
            mask = m.to(self.device)
        out = self.model.decode_step(input_ids=ids, past_key_values=cache, encoder_past_kv_list=enc_list,
                                     attention_mask=mask, encoder_attention_mask=enc_mask, position_ids=pos,
                                     use_cache=True)
        slots = torch.tensor([dec_bm.slot(r.decoder_block_table, r.decoder_seq_len) for r in run],
                             dtype=torch.int64).to(self.device)
        for l in range(dec_bm.num_layers):
            layer = out.past_key_values.layers[l]
            native.append(layer.keys[:, :, -1, :], layer.values[:, :, -1, :], dec_bm.key_pool[l],
                          dec_bm.value_pool[l], slots)
        return out

    def _process_decode_phase_graph(self) -> None:
        gb = self.graph_buffers
        t0 = time.perf_counter()
        bucket = gb.prepare_replay()
        gb.replay_step(bucket)
        self.decode_steps += 1
        if gb.should_readback():
            results = gb.sync_tokens()
            done = []
            for slot, tokens in results:
                req = slot.req
                for off, (tok, trace) in enumerate(zip(tokens, slot.last_readback_trace)):
                    if req.done:
                        break
                    req.graph_token_trace.append({"token_index": len(req.generated_tokens),
                                                  "bucket": trace["bucket"],
                                                  "readback_position": trace["readback_position"]})
                    req.last_token_id = tok
                    req.generated_tokens.append(tok)
                    req.generated_count = len(req.generated_tokens)
                    req.decoder_seq_len = req.prompt_token_ids.shape[-1] + req.generated_count
                    is_eos = req.eos_token_id is not None and tok == req.eos_token_id
                    if is_eos or req.generated_count >= req.max_new_tokens:
                        req.graph_extra_slot_steps = len(tokens) - off - 1
                        if is_eos and req.eos_token_id in req.generated_tokens:
                            req.generated_tokens = req.generated_tokens[:req.generated_tokens.index(req.eos_token_id)]
                        gb.release_slot(slot.slot_idx)
                        req.slot_idx = None
                        self._complete_request(req, status=RequestPhase.COMPLETED)
                        done.append(req)
                        break
            if done:
                self.active_decode = [r for r in self.active_decode if r not in done]
        self.decode_time_s += time.perf_counter() - t0

    # ------------------------------------------------------------------ completion
    def _complete_request(self, req: DualCacheRequest, status: RequestPhase) -> None:
        """Release decoder blocks, encoder blocks, the cross slot and the graph slot."""
        req.phase = status
        req.done = True
        req.finish_time = time.perf_counter()
        if self.graph_decode and req.slot_idx is not None:
            self.graph_buffers.release_slot(req.slot_idx)
            req.slot_idx = None
        try:
            if req.decoder_block_table:
                self.dual_cache.decoder_bm.free_blocks(req.decoder_block_table)
                req.decoder_block_table = []
            if req.encoder_block_table:
                self.dual_cache.encoder_bm.release_blocks(req.encoder_block_table)
                if not self.retain_encoder_cache and req.full_input_hash in self._full_input_enc_cache:
                    entry = self._full_input_enc_cache[req.full_input_hash]
                    if all(self.dual_cache.encoder_bm.ref_counts[b] == 0 for b in entry["block_table"]):
                        self._full_input_enc_cache.pop(req.full_input_hash, None)
                req.encoder_block_table = []
            if self.cross_arena is not None:
                self.cross_arena.release(req)
        finally:
            req.cached_decoder_kv = None
            req.cached_encoder_kv = None
            self.completed.append(req)

    # ------------------------------------------------------------------ loop
    def _update_peak_actually_used(self) -> None:
        dec = self.dual_cache.decoder_bm
        enc = self.dual_cache.encoder_bm
        used = dec.allocated_block_count * dec.block_bytes() + enc.allocated_block_count * enc.bytes_per_block
        self.peak_pool_blocks_used_bytes = max(self.peak_pool_blocks_used_bytes, used)
        self.peak_actually_used_bytes = max(self.peak_actually_used_bytes, used)

    def step(self) -> bool:
        in_flight = len(self.active_encode) + len(self.active_decode)
        self.peak_in_flight_requests = max(self.peak_in_flight_requests, in_flight)
        self.in_flight_history.append(in_flight)
        self._update_peak_actually_used()
        if self.verbose:
            self.memory_guard.log_telemetry(in_flight, len(self.queue), self.dual_cache.encoder_bm.get_stats(),
                                            self.dual_cache.decoder_bm.get_stats())
        self._process_encode_phase()
        self._update_peak_actually_used()
        self._process_decode_phase()
        self._update_peak_actually_used()
        if self.step_delay > 0:
            time.sleep(self.step_delay)
        return self.has_work()

    def has_work(self) -> bool:
        return bool(self.queue or self.active_encode or self.active_decode)

    def run_until_done(self, max_steps: int = 100000) -> List[DualCacheRequest]:
        steps = 0
        while self.step() and steps < max_steps:
            steps += 1
        return self.completed

    # ------------------------------------------------------------------ telemetry
    def reset_telemetry(self) -> None:
        self.encoder_calls = 0
        self.encoder_calls_skipped = 0
        self.encode_time_saved_s = 0.0
        self.rejected_requests_count = 0
        self.in_flight_history = []
        self.queue_wait_times = []
        self.completed = []
        self.peak_in_flight_requests = 0
        self.peak_actually_used_bytes = 0
        self.decode_steps = 0
        self.decode_time_s = 0.0

    def get_concurrency_stats(self) -> Dict[str, Any]:
        enc, dec = self.dual_cache.encoder_bm, self.dual_cache.decoder_bm
        enc_blk, dec_blk = enc.bytes_per_block, dec.block_bytes()
        q = self.queue_wait_times or [0.0]
        inf = self.in_flight_history or [0]
        return {
            "encoder_pool_blocks": enc.num_blocks,
            "encoder_pool_mb": enc.num_blocks * enc_blk / 2 ** 20,
            "decoder_pool_blocks": dec.num_blocks,
            "decoder_pool_mb": dec.num_blocks * dec_blk / 2 ** 20,
            "total_pool_mb": (enc.num_blocks * enc_blk + dec.num_blocks * dec_blk) / 2 ** 20,
            "req_encoder_blocks": -(-1500 // enc.block_size),
            "req_encoder_mb": -(-1500 // enc.block_size) * enc_blk / 2 ** 20,
            "req_decoder_blocks": -(-150 // dec.block_size),
            "req_decoder_mb": -(-150 // dec.block_size) * dec_blk / 2 ** 20,
            "avg_in_flight_requests": float(np.mean(inf)),
            "max_in_flight_requests": int(max(inf)),
            "queue_wait_time_mean_s": float(np.mean(q)),
            "queue_wait_time_p50_s": float(np.percentile(q, 50)),
            "queue_wait_time_p95_s": float(np.percentile(q, 95)),
            "rejections_per_run": self.rejected_requests_count,
            "peak_actually_used_mb": self.peak_actually_used_bytes / 2 ** 20,
        }

    def get_encoder_telemetry(self) -> Dict[str, Any]:
        total = self.encoder_calls + self.encoder_calls_skipped
        return {
            "encoder_calls": self.encoder_calls,
            "encoder_calls_skipped": self.encoder_calls_skipped,
            "encode_time_saved_s": round(self.encode_time_saved_s, 4),
            "total_requests": total,
            "skip_rate_pct": round(self.encoder_calls_skipped / total * 100.0, 2) if total else 0.0,
            "full_input_cache_entries": len(self._full_input_enc_cache),
            "max_cached_encoder_inputs": self.max_cached_encoder_inputs,
        }
