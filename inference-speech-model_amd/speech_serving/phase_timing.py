"""Opt-in per-request phase timer (interface of the reference's PhaseTimer,
speech_serving/phase_timing.py:34-86). When enabled it synchronises the
device at phase boundaries and accumulates wall milliseconds per phase."""
from __future__ import annotations

import contextlib
import time
from typing import Any, Dict, Iterable

import torch


class PhaseTimer:
    def __init__(self, enabled: bool = False, device: str = "cuda"):
        self.enabled = bool(enabled)
        self.device = device

    def ensure(self, req) -> Dict[str, Any]:
        if req.phase_timing is None:
            req.phase_timing = {}
        return req.phase_timing

    def add(self, reqs: Iterable[Any], name: str, ms: float, gpu_ms: float = 0.0) -> None:
        if not self.enabled:
            return
        for r in reqs:
            pt = self.ensure(r)
            pt[name] = pt.get(name, 0.0) + ms

    @contextlib.contextmanager
    def measure(self, reqs, name: str):
        if not self.enabled:
            yield
            return
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        try:
            yield
        finally:
            if torch.cuda.is_available():
                torch.cuda.synchronize()
            self.add(list(reqs), name, (time.perf_counter() - t0) * 1e3)
