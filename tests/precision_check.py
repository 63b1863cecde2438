"""Greedy-token parity of fp16/bf16 GPU decoding against the float64 oracle (test helper).

The oracle decodes with the GPU model's own rounded weights and encoder K/V (cast to float64), so
every difference comes from the GPU's reduced-precision arithmetic: activations, K/V and logits
rounded to the dtype, fp32 accumulation. Both sides are teacher-forced along one token path (the
GPU's greedy tokens), so a near-tie at one step does not change the context of the next.

Bar. Let E bound the GPU's logit error against the oracle on that path:
    E = 8 * u * sqrt(L) * rms(oracle logits of the step)
with u the dtype's unit roundoff (fp16 2^-11, bf16 2^-8) and L the decoder layers: one rounding of
the residual stream per sub-layer accumulates as a random walk over the layers, and the final
LayerNorm maps it onto the logits at their own scale. (Measured on MI355X: the largest error is
5.2 u sqrt(L) rms at the base shape in fp16, 4.4 at the small shape and 4.0 at the large-v3 shape in
bf16.) Then at every step
  * max |logits_gpu - logits_oracle| <= E (where the GPU logits are available), and
  * the GPU's token t satisfies oracle[t] >= max(oracle) - 2E: it is the oracle's argmax whenever the
    oracle's top-2 margin exceeds 2E, and within 2E of it at a near-tie.
float32 decoding is held to the reference's golden vectors and the oracle's tokens directly instead.
The reference path being followed is speech_serving/phase_aware_scheduler.py:771-1044 (eager greedy
loop) and the sequential-vs-batched check of test_speech_engine.py:237-298.
"""
from __future__ import annotations

import math
from typing import Dict, List, Sequence, Tuple

import numpy as np
import torch

from oracle import decoder as D
from speech_serving.block_manager import BlockManager
from speech_serving.models import CrossKV, PagedKV

UNIT_ROUNDOFF = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def oracle_of(m) -> D.Model:
    """The float64 oracle on the GPU model's (rounded) weights."""
    state = {k: v.detach().float().cpu().numpy() for k, v in m.state_dict().items()}
    return D.Model(state, m.num_heads, m.head_dim)


def error_bound(dtype: torch.dtype, layers: int, oracle_logits: np.ndarray) -> np.ndarray:
    """E per step (oracle_logits [..., V] -> [...])."""
    rms = np.sqrt((oracle_logits ** 2).mean(axis=-1))
    return 8.0 * UNIT_ROUNDOFF[dtype] * math.sqrt(layers) * rms


def oracle_logits_along(om: D.Model, prompt: Sequence[int], cross: Sequence[Sequence[Tuple[np.ndarray, np.ndarray]]],
                        paths: Sequence[Sequence[int]], steps: int) -> np.ndarray:
    """Teacher-forced float64 logits [R, steps, V]: step 0 is the prompt's last position, step s > 0
    follows paths[r][:s]. cross[r] is request r's per-layer (K, V) [1, H, T_r, D]; requests with
    the same T run as one batch."""
    out = [None] * len(paths)
    groups: Dict[int, List[int]] = {}
    for r, c in enumerate(cross):
        groups.setdefault(c[0][0].shape[2], []).append(r)
    for rs in groups.values():
        ck = [(np.concatenate([cross[r][l][0] for r in rs]), np.concatenate([cross[r][l][1] for r in rs]))
              for l in range(len(cross[rs[0]]))]
        logits, past = om.decode_step(np.asarray([list(prompt)] * len(rs)), None, ck)
        got = [logits[:, -1]]
        for s in range(1, steps):
            ids = np.asarray([[paths[r][s - 1]] for r in rs])
            logits, past = om.decode_step(ids, past, ck)
            got.append(logits[:, -1])
        stacked = np.stack(got, axis=1)
        for i, r in enumerate(rs):
            out[r] = stacked[i]
    return np.stack(out)


def gpu_logits_along(m, prompt: Sequence[int], kvs: Sequence[Sequence[Tuple[torch.Tensor, torch.Tensor]]],
                     paths: Sequence[Sequence[int]], steps: int, free_running: bool = False) -> np.ndarray:
    """Teacher-forced GPU logits [R, steps, V] through the eager paged decode (prefill with the
    fused causal append, then one token per step), the requests batched in one decode. With
    free_running the path is the GPU's own greedy tokens, written into paths (lists)."""
    dev = m.decoder_norm.weight.device
    dt = m.decoder_norm.weight.dtype
    r_n = len(paths)
    bs = 16
    per = -(-(len(prompt) + steps) // bs)
    dec = BlockManager(m.num_decoder_layers, m.num_heads, m.head_dim, bs, r_n * per, dtype=dt, device=str(dev))
    tables = torch.tensor([[dec.allocate_block() for _ in range(per)] for _ in range(r_n)], dtype=torch.int32,
                          device=dev)
    t_max = max(kv[0][0].shape[2] for kv in kvs)
    layers = m.num_decoder_layers
    ck, cv = [], []
    for l in range(layers):
        k = torch.zeros(r_n, m.num_heads, t_max, m.head_dim, dtype=dt, device=dev)
        v = torch.zeros_like(k)
        for r, kv in enumerate(kvs):
            t = kv[l][0].shape[2]
            k[r, :, :t] = kv[l][0][0]
            v[r, :, :t] = kv[l][1][0]
        ck.append(k)
        cv.append(v)
    lens = torch.tensor([kv[0][0].shape[2] for kv in kvs], dtype=torch.int32, device=dev)
    cross = CrossKV(ck, cv, lens, t_max)
    p = len(prompt)
    out = []
    with torch.no_grad():
        ids = torch.tensor([list(prompt)] * r_n, device=dev)
        for s in range(steps):
            n = p + s
            kv = PagedKV(dec.key_pool, dec.value_pool, tables, torch.full((r_n,), n, dtype=torch.int32, device=dev), n)
            logits = m.decode_step_paged(ids, kv, cross)
            out.append(logits.float().cpu().numpy())
            if free_running:
                for r, t in enumerate(logits.argmax(-1).tolist()):
                    paths[r].append(t)
            if s + 1 < steps:
                ids = torch.tensor([[paths[r][s]] for r in range(r_n)], device=dev)
    return np.stack(out, axis=1)


def check_tokens(dtype: torch.dtype, layers: int, oracle_logits: np.ndarray, paths: Sequence[Sequence[int]],
                 gpu_logits: np.ndarray = None) -> dict:
    """Assert the bar of this module on R requests x S steps; returns what was compared."""
    steps = oracle_logits.shape[1]
    e = error_bound(dtype, layers, oracle_logits)  # [R, S]
    tok = np.asarray([list(p[:steps]) for p in paths])  # [R, S]
    top2 = np.sort(oracle_logits, axis=-1)[..., -2:]
    margin = top2[..., 1] - top2[..., 0]
    slack = oracle_logits.max(axis=-1) - np.take_along_axis(oracle_logits, tok[..., None], axis=-1)[..., 0]
    stats = {"requests": len(paths), "steps": steps, "max_E": float(e.max()),
             "near_ties": int((margin <= 2 * e).sum()), "argmax_equal": int((slack == 0).sum()),
             "max_slack_over_2E": float((slack / (2 * e)).max())}
    if gpu_logits is not None:
        err = np.abs(gpu_logits - oracle_logits).max(axis=-1)
        stats["max_err_over_E"] = float((err / e).max())
        stats["max_logit_err"] = float(err.max())
        assert (err <= e).all(), f"GPU logits differ from the float64 oracle by more than E: {stats}"
    assert (slack <= 2 * e).all(), f"a GPU token is not within 2E of the oracle's maximum: {stats}"
    assert ((margin <= 2 * e) | (slack == 0)).all(), f"GPU token differs from the oracle's clear argmax: {stats}"
    return stats
