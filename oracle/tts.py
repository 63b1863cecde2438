"""numpy oracle of the streaming multi-codebook TTS model and engine (float64).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Restates, from the
reference's source text (paths relative to the reference repository):
    embed              MultiCodebookEmbedding.forward, speech_serving/models.py:38-51
                       (sum of the K codebooks' embedding rows)
    heads              MultiCodebookHeads.forward, models.py:69-77 (one bias-free
                       Linear per codebook, stacked on axis 2)
    TTSModel.forward   StreamingMultiCodebookTTSModel.forward, models.py:251-295:
                       embed, DecoderLayer.forward per layer without cross-attention
                       (so the MLP normalises with norm2, models.py:206), final
                       LayerNorm, heads
    TTSModel.generate  one request through StreamingTTSEngine: prefill and first
                       frame (tts_engine.py:95-140), then one frame per step from
                       the request's whole past (tts_engine.py:166-215); argmax
                       per codebook, first maximum on ties
    Engine             the engine's admission, block allocation and release order
                       (tts_engine.py:95-152, 154-239) over a LIFO free list
                       (block_manager.py:133-166)
Pinned by tests/golden/tts_small_golden.npz (written from the reference
implementation) and by invariants in tests/test_tts_oracle.py.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from .decoder import F64, Model, layer_norm, linear


class TTSModel:
    def __init__(self, state: Dict[str, np.ndarray], num_heads: int, head_dim: int):
        self.core = Model(state, num_heads, head_dim)  # DecoderLayer.forward restatement
        self.p = self.core.p
        self.n_layers = len({k.split(".")[1] for k in state if k.startswith("layers.")})
        self.n_cb = len({k.split(".")[2] for k in state if k.startswith("embeddings.embeddings.")})

    def embed(self, codes: np.ndarray) -> np.ndarray:
        """codes [B, S, K] -> [B, S, hidden]: sum over k of E_k[codes[..., k]]."""
        codes = np.asarray(codes)
        x = self.p["embeddings.embeddings.0.weight"][codes[..., 0]]
        for k in range(1, self.n_cb):
            x = x + self.p[f"embeddings.embeddings.{k}.weight"][codes[..., k]]
        return x

    def heads(self, x: np.ndarray) -> np.ndarray:
        """[B, S, hidden] -> logits [B, S, K, V]."""
        return np.stack([linear(x, self.p[f"heads.heads.{k}.weight"]) for k in range(self.n_cb)], axis=2)

    def forward(self, codes: np.ndarray, past: Optional[List[Tuple[np.ndarray, np.ndarray]]] = None):
        """logits [B, S, K, V] and the per-layer (K, V) [B, H, T, D] including the new positions."""
        x = self.embed(codes)
        new = []
        for i in range(self.n_layers):
            x, kv = self.core.layer(f"layers.{i}", x, past[i] if past is not None else None, None, is_decoder=True)
            new.append(kv)
        x = layer_norm(x, self.p["norm.weight"], self.p["norm.bias"])
        return self.heads(x), new

    def generate(self, prompt: np.ndarray, frames: int) -> Tuple[np.ndarray, np.ndarray]:
        """prompt [P, K] -> (frames [F, K], last-position logits [F, K, V])."""
        logits, past = self.forward(np.asarray(prompt)[None])
        out, lg = [], []
        while True:
            last = logits[0, -1]
            lg.append(last)
            tok = last.argmax(axis=-1)
            out.append(tok)
            if len(out) >= frames:
                return np.stack(out).astype(np.int64), np.stack(lg)
            logits, past = self.forward(tok[None, None], past)


class Engine:
    """Block bookkeeping of StreamingTTSEngine over a LIFO free list: which blocks each
    request holds when, and the order requests complete in. Frames come from TTSModel."""

    def __init__(self, num_blocks: int, block_size: int, max_batch: int):
        self.free = list(range(num_blocks))
        self.bs = block_size
        self.max_batch = max_batch

    def run(self, prompt_lens: Sequence[int], max_new_frames: Sequence[int]):
        """Returns (completion order, per request the list of its block tables after each
        frame it produced, peak number of allocated blocks)."""
        queue = list(range(len(prompt_lens)))
        active: List[int] = []
        seq = {}
        table: Dict[int, List[int]] = {}
        count = {}
        history: Dict[int, List[List[int]]] = {r: [] for r in queue}
        done: List[int] = []
        peak = 0
        n_total = len(self.free)

        def finish(r):
            self.free.extend(table[r])  # free_blocks appends in table order (block_manager.py:152-166)
            table[r] = []
            done.append(r)

        while active or queue:
            # admission (tts_engine.py:95-152)
            while len(active) < self.max_batch and queue:
                r = queue.pop(0)
                seq[r] = prompt_lens[r]
                table[r] = [self.free.pop() for _ in range((seq[r] + self.bs - 1) // self.bs)]
                peak = max(peak, n_total - len(self.free))
                count[r] = 1
                history[r].append(list(table[r]))
                if count[r] >= max_new_frames[r]:
                    finish(r)
                else:
                    active.append(r)
            if not active:
                break
            # one decode step (tts_engine.py:154-239)
            still = []
            for r in active:
                if seq[r] % self.bs == 0:
                    table[r].append(self.free.pop())
                    peak = max(peak, n_total - len(self.free))
                seq[r] += 1
                count[r] += 1
                history[r].append(list(table[r]))
                if count[r] >= max_new_frames[r]:
                    finish(r)
                else:
                    still.append(r)
            active = still
        return done, history, peak
