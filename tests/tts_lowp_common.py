"""The reference's fp16 / bf16 streaming TTS decodes (tests/golden/tts_lowp_golden.npz) and their error
model (test helper).

Each fixture entry is one request of the reference's own reduced-precision decode (its
StreamingMultiCodebookTTSModel cast to float16 or bfloat16 on the CPU, model(...) with a DynamicCache per
frame, argmax per codebook; tests/golden/make_tts_golden.py --lowp): the prompt frames, and per generated
frame its K codes and each codebook's top-16 logits. Weights are regenerated here from the seed
(oracle/rounding.seeded_state) and checked against the fixture's checksums.

A frame has K heads, so a (frame, codebook) pair is one row of the comparison: its logits are head k's
[V] vector at that position, its token the frame's code k. Bars are those of lowp_common (the derived
rounding model of oracle/rounding.py over the MultiCodebook64 restatement, K_SIGMA sigma), applied per row.
"""
from __future__ import annotations

import json
import os
from typing import Dict, List, Tuple

import numpy as np
import torch

from lowp_common import DTYPES, K_SIGMA, compare  # noqa: F401  (compare: re-exported for the tests)
from oracle.rounding import MultiCodebook64, checksums, rounding_sigma, seeded_state

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tts_lowp_golden.npz")


def load():
    z = np.load(GOLDEN, allow_pickle=False)
    return z, json.loads(bytes(z["config_json"]).decode())


def cases(cfg) -> List[Tuple[str, str]]:
    return [(shape, dname) for shape in cfg["shapes"] for dname in DTYPES]


def model_args(c) -> Dict[str, int]:
    return {k: c[k] for k in ("num_layers", "num_heads", "hidden_dim", "num_codebooks", "vocab_size")}


def model_state(shape_cfg, state_names: Dict[str, Tuple[int, ...]], dtype) -> Dict[str, torch.Tensor]:
    st = seeded_state(state_names, shape_cfg["seed"], shape_cfg["std"])
    return {k: v.to(dtype) for k, v in st.items()}


def check_state(z, shape: str, dname: str, state: Dict[str, torch.Tensor]) -> None:
    assert np.array_equal(checksums(state).numpy(), z[f"{shape}.{dname}.param_checksums"]), \
        f"{shape}.{dname}: regenerated weights differ from the fixture's"


class TTSReference:
    """One fixture request along the reference's frame path, as rows (frame, codebook), with the error
    model of a comparison against it: the targets are the reference's logits (the fixture), or with
    float64=True float64 math along the same path. sigma sums the rounding sites of `placements`."""

    def __init__(self, z, shape_cfg, key: str, model: MultiCodebook64, dtype, placements, float64: bool = False):
        c = shape_cfg
        k_n, v_n = c["num_codebooks"], c["vocab_size"]
        self.prompt = z[f"{key}.prompt"].tolist()
        self.frames = z[f"{key}.frames"].tolist()
        f_n = len(self.frames)
        self.seq = self.prompt + self.frames[:-1]  # the teacher-forced frames
        p = len(self.prompt)
        pos = [p - 1 + t for t in range(f_n)]
        if float64:
            l64 = model.forward(self.seq, None)[pos].detach().numpy().reshape(f_n * k_n, v_n)
            self.top_idx = np.argsort(-l64, axis=1, kind="stable")[:, :16]
            self.top_val = np.take_along_axis(l64, self.top_idx, axis=1)
            self.tokens = [int(i) for i in self.top_idx[:, 0]]
        else:
            self.tokens = [int(t) for f in self.frames for t in f]
            self.top_idx = z[f"{key}.topk_idx"].reshape(f_n * k_n, -1)
            self.top_val = z[f"{key}.topk_val"].reshape(f_n * k_n, -1).astype(np.float64)
        rows_pos = [pt for pt in pos for _ in range(k_n)]
        a = [k * v_n + int(self.top_idx[r, 0]) for r, k in zip(range(f_n * k_n), list(range(k_n)) * f_n)]
        b = [k * v_n + int(self.top_idx[r, 1]) for r, k in zip(range(f_n * k_n), list(range(k_n)) * f_n)]
        sm, logits64 = rounding_sigma(model, self.seq, None, dtype, rows_pos, list(zip(a, b)), placements)
        st, _ = rounding_sigma(model, self.seq, None, dtype, rows_pos, [(x, None) for x in a], placements)
        self.sigma_margin, self.sigma_top = sm.numpy(), st.numpy()
        self.logits64 = logits64[pos].numpy().reshape(f_n * k_n, v_n)  # float64 logits per row
        self.margin = self.top_val[:, 0] - self.top_val[:, 1]
        self.near_tie = self.margin <= K_SIGMA * self.sigma_margin
        self.k_n = k_n
