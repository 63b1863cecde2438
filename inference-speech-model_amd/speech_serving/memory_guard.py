"""High-water-mark admission guard and eviction telemetry.

Interface of the reference's MemoryGuard (speech_serving/memory_guard.py:20-99).
"""
from __future__ import annotations

import logging
import time
from typing import Any, Dict

import torch

logger = logging.getLogger("SpeechMemoryGuard")


class MemoryGuard:
    def __init__(self, high_water_mark_pct: float = 90.0, enable_periodic_gc: bool = True):
        self.high_water_mark_pct = high_water_mark_pct
        self.enable_periodic_gc = enable_periodic_gc
        self.eviction_events_count = 0
        self.last_empty_cache_time = time.perf_counter()
        self.total_freed_blocks_count = 0

    def check_high_water_mark(self, encoder_allocated: int, encoder_total: int, decoder_allocated: int,
                              decoder_total: int) -> bool:
        total = encoder_total + decoder_total
        if total == 0:
            return False
        util = (encoder_allocated + decoder_allocated) / total * 100.0
        if util >= self.high_water_mark_pct:
            logger.warning("KV block pools at %.1f%% of capacity (admission limit %.1f%%)", util,
                           self.high_water_mark_pct)
            return True
        return False

    def trigger_bulk_eviction_cleanup(self, freed_blocks: int, reason: str = "high_water_mark"):
        self.eviction_events_count += 1
        self.total_freed_blocks_count += freed_blocks
        logger.info("eviction %d (%s): %d blocks returned to the pools", self.eviction_events_count, reason,
                    freed_blocks)
        if self.enable_periodic_gc and torch.cuda.is_available():
            torch.cuda.empty_cache()
            self.last_empty_cache_time = time.perf_counter()

    def log_telemetry(self, active_requests: int, queued_requests: int, encoder_stats: Dict[str, Any],
                      decoder_stats: Dict[str, Any]):
        logger.info("requests: %d decoding, %d waiting; encoder pool %s%% used, decoder pool %s%% used; "
                    "%d evictions so far", active_requests, queued_requests, encoder_stats["utilization_pct"],
                    decoder_stats["utilization_pct"], self.eviction_events_count)
