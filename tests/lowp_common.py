"""The reference's fp16 / bf16 greedy decodes (tests/golden/whisper_lowp_golden.npz) and their error model
(test helper).

Each fixture entry is one request of the reference's own reduced-precision decode (its model cast to
float16 or bfloat16 on the CPU, decode_step with a DynamicCache, torch.argmax per step;
tests/golden/make_golden.py --lowp): per step the token and the top-16 logits. Weights and encoder K/V
are regenerated here from the same seeds (oracle/rounding.seeded_state / seeded_cross_kv) and checked
against the fixture's checksums.

Bars come from oracle/rounding.rounding_sigma, the first-order rounding-error model (no constant fitted
to measurements): sigma(z) of a logit, or of the top-2 margin, sums ulp^2/12 x sensitivity^2 over the
rounding sites of the implementations being compared. A comparison passes within K_SIGMA = 5 sigma.
"""
from __future__ import annotations

import json
import os
from typing import Dict, List, Tuple

import numpy as np
import torch

from oracle.rounding import Decoder64, checksums, rounding_sigma, seeded_cross_kv, seeded_state

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "whisper_lowp_golden.npz")
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}
K_SIGMA = 5.0


def load():
    z = np.load(GOLDEN, allow_pickle=False)
    return z, json.loads(bytes(z["config_json"]).decode())


def cases(cfg) -> List[Tuple[str, str]]:
    return [(shape, dname) for shape in cfg["shapes"] for dname in DTYPES]


def model_state(shape_cfg, state_names: Dict[str, Tuple[int, ...]], dtype) -> Dict[str, torch.Tensor]:
    st = seeded_state(state_names, shape_cfg["seed"], shape_cfg["std"])
    return {k: v.to(dtype) for k, v in st.items()}


def cross_kv(shape_cfg, r: int, dtype) -> List[Tuple[torch.Tensor, torch.Tensor]]:
    c = shape_cfg
    return [(k.to(dtype), v.to(dtype)) for k, v in
            seeded_cross_kv(c["layers"], c["heads"], c["t_enc"], c["head_dim"], c["kv_seeds"][r], c["kv_std"])]


def check_inputs(z, shape: str, dname: str, state: Dict[str, torch.Tensor], crosses) -> None:
    assert np.array_equal(checksums(state).numpy(), z[f"{shape}.{dname}.param_checksums"]), \
        f"{shape}.{dname}: regenerated weights differ from the fixture's"
    for r, cross in enumerate(crosses):
        got = checksums({f"{l}.{j}": t for l, kv in enumerate(cross) for j, t in enumerate(kv)}).numpy()
        assert np.array_equal(got, z[f"{shape}.{dname}.r{r}.kv_checksums"]), f"{shape}.{dname}.r{r}: encoder K/V"


class Reference:
    """One fixture request along the reference's token path, with the error model of a comparison against it.

    The targets are the reference's logits (the fixture: its tokens and top-16 logits), or, with
    float64=True, float64 math along the same path (argmax and top-16 of Decoder64's logits). sigma sums
    the rounding sites of `placements`: ("reference", "paged") for the paged path against the reference,
    ("paged",) for the paged path against float64, ("reference",) for the reference against float64."""

    def __init__(self, z, shape_cfg, key: str, dec: Decoder64, cross, dtype, placements, float64: bool = False):
        c = shape_cfg
        path = z[f"{key}.tokens"].tolist()
        self.prompt = list(c["prompt"])
        self.ids = self.prompt + path[:-1]  # the teacher-forced sequence
        p = len(self.prompt)
        self.positions = [p - 1 + i for i in range(len(path))]
        if float64:
            self.logits64 = dec.forward(self.ids, cross)[self.positions].detach().numpy()
            self.top_idx = np.argsort(-self.logits64, axis=1, kind="stable")[:, :16]
            self.top_val = np.take_along_axis(self.logits64, self.top_idx, axis=1)
            self.tokens = [int(i) for i in self.top_idx[:, 0]]
        else:
            self.tokens = path
            self.top_idx = z[f"{key}.topk_idx"]
            self.top_val = z[f"{key}.topk_val"].astype(np.float64)
        a = [int(i) for i in self.top_idx[:, 0]]
        b = [int(i) for i in self.top_idx[:, 1]]
        sm, logits64 = rounding_sigma(dec, self.ids, cross, dtype, self.positions, list(zip(a, b)), placements)
        st, _ = rounding_sigma(dec, self.ids, cross, dtype, self.positions, [(x, None) for x in a], placements)
        self.sigma_margin, self.sigma_top = sm.numpy(), st.numpy()
        self.logits64 = logits64[self.positions].numpy()  # [steps, V] float64 logits along the path
        self.margin = self.top_val[:, 0] - self.top_val[:, 1]
        self.near_tie = self.margin <= K_SIGMA * self.sigma_margin


def compare(ref: Reference, logits: np.ndarray, what: str) -> Dict[str, int]:
    """logits [steps, V] of another implementation along ref's path, against the reference's: the top-1 logit
    and the top-2 margin within K_SIGMA sigma; the argmax equal to the reference's token except at a near-tie,
    where it must be a token the reference's logits put within K_SIGMA sigma of the maximum."""
    steps = len(ref.tokens)
    eq = 0
    for s in range(steps):
        a, b = int(ref.top_idx[s, 0]), int(ref.top_idx[s, 1])
        top = logits[s, a]
        assert abs(top - ref.top_val[s, 0]) <= K_SIGMA * ref.sigma_top[s], \
            f"{what} step {s}: logit {top:.6f} vs the reference's {ref.top_val[s, 0]:.6f} (sigma {ref.sigma_top[s]:.2e})"
        m = logits[s, a] - logits[s, b]
        assert abs(m - ref.margin[s]) <= K_SIGMA * ref.sigma_margin[s], \
            f"{what} step {s}: margin {m:.6f} vs {ref.margin[s]:.6f} (sigma {ref.sigma_margin[s]:.2e})"
        t = int(np.argmax(logits[s]))
        if t == ref.tokens[s]:
            eq += 1
        else:
            assert ref.near_tie[s], f"{what} step {s}: token {t} vs the reference's {ref.tokens[s]} " \
                                    f"(margin {ref.margin[s]:.3e} > {K_SIGMA} sigma {ref.sigma_margin[s]:.2e})"
            hit = np.nonzero(ref.top_idx[s] == t)[0]
            assert hit.size and ref.top_val[s, hit[0]] >= ref.top_val[s, 0] - K_SIGMA * ref.sigma_margin[s], \
                f"{what} step {s}: token {t} is not among the reference's near-tied tokens"
    return {"steps": steps, "argmax_equal": eq, "near_ties": int(ref.near_tie.sum())}
