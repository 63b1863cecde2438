"""numpy oracle of the synthetic Whisper-class encoder-decoder (float64).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Restates, from the
reference's source text (paths relative to the reference repository):
    layer_norm, gelu   torch.nn.LayerNorm (eps 1e-5) and nn.GELU (exact erf form)
    conv1d             torch.nn.Conv1d (kernel 3, padding 1, stride 1 / 2)
    Layer.forward      speech_serving/models.py:110-208 (pre-LN self-attention
                       with causal triu mask for multi-token decoder input,
                       optional cross-attention, MLP on norm3 when cross-
                       attention ran, else norm2)
    Model.encode       speech_serving/models.py:349-367
    Model.decode_step  speech_serving/models.py:369-423 (one request, B = 1)
    Model.greedy       the sequential reference loop of test_speech_engine.py
                       :264-280 with the scheduler's EOS rule
                       (phase_aware_scheduler.py:692-703, 1022-1036)
Weights come from a state_dict with the reference's parameter names.
Pinned by tests/golden/ vectors written from the reference implementation.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
from scipy.special import erf

F64 = np.float64


def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def gelu(x: np.ndarray) -> np.ndarray:
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def linear(x: np.ndarray, w: np.ndarray, b: Optional[np.ndarray] = None) -> np.ndarray:
    y = x @ w.T
    return y if b is None else y + b


def conv1d(x: np.ndarray, w: np.ndarray, b: np.ndarray, stride: int, padding: int) -> np.ndarray:
    """x [B, C_in, L], w [C_out, C_in, K] -> [B, C_out, L_out] (cross-correlation)."""
    bsz, cin, n = x.shape
    cout, _, k = w.shape
    xp = np.pad(x, ((0, 0), (0, 0), (padding, padding)))
    lout = (n + 2 * padding - k) // stride + 1
    cols = np.stack([xp[:, :, i * stride:i * stride + k] for i in range(lout)], axis=2)  # [B, C_in, L_out, K]
    return np.einsum("bclk,ock->bol", cols, w) + b[None, :, None]


def softmax(s: np.ndarray) -> np.ndarray:
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


class Model:
    def __init__(self, state: Dict[str, np.ndarray], num_heads: int, head_dim: int):
        self.p = {k: np.asarray(v, dtype=F64) for k, v in state.items()}
        self.h = num_heads
        self.d = head_dim
        self.n_enc = len({k.split(".")[1] for k in state if k.startswith("encoder_layers.")})
        self.n_dec = len({k.split(".")[1] for k in state if k.startswith("decoder_layers.")})

    def _heads(self, x: np.ndarray) -> np.ndarray:
        b, s, _ = x.shape
        return x.reshape(b, s, self.h, self.d).transpose(0, 2, 1, 3)  # [B, H, S, D]

    def layer(self, prefix: str, x: np.ndarray, past: Optional[Tuple[np.ndarray, np.ndarray]] = None,
              cross: Optional[Tuple[np.ndarray, np.ndarray]] = None, is_decoder: bool = True):
        """models.py:110-208 for one layer; x [B, S, hidden]. Returns x, (k, v)."""
        P = lambda n: self.p[f"{prefix}.{n}"]  # noqa: E731
        b, s, _ = x.shape
        scale = 1.0 / math.sqrt(self.d)
        h1 = layer_norm(x, P("norm1.weight"), P("norm1.bias"))
        q = self._heads(linear(h1, P("self_attn_q.weight")))
        k = self._heads(linear(h1, P("self_attn_k.weight")))
        v = self._heads(linear(h1, P("self_attn_v.weight")))
        if past is not None:
            k = np.concatenate([past[0], k], axis=2)
            v = np.concatenate([past[1], v], axis=2)
        w = np.einsum("bhqd,bhtd->bhqt", q, k) * scale
        if is_decoder and s > 1:
            w = w + np.triu(np.full((s, k.shape[2]), -np.inf), k=1)
        o = np.einsum("bhqt,bhtd->bhqd", softmax(w), v).transpose(0, 2, 1, 3).reshape(b, s, -1)
        x = x + linear(o, P("self_attn_out.weight"))
        used = cross is not None
        if used:
            h2 = layer_norm(x, P("norm2.weight"), P("norm2.bias"))
            cq = self._heads(linear(h2, P("cross_attn_q.weight")))
            ck, cv = cross
            cw = np.einsum("bhqd,bhtd->bhqt", cq, ck) * scale
            co = np.einsum("bhqt,bhtd->bhqd", softmax(cw), cv).transpose(0, 2, 1, 3).reshape(b, s, -1)
            x = x + linear(co, P("cross_attn_out.weight"))
        n = "norm3" if used else "norm2"
        hm = layer_norm(x, P(f"{n}.weight"), P(f"{n}.bias"))
        m = linear(gelu(linear(hm, P("mlp.0.weight"), P("mlp.0.bias"))), P("mlp.2.weight"), P("mlp.2.bias"))
        return x + m, (k, v)

    def encode(self, mel: np.ndarray):
        """models.py:349-367; mel [B, mel_dim, L]."""
        x = gelu(conv1d(np.asarray(mel, F64), self.p["conv1.weight"], self.p["conv1.bias"], 1, 1))
        x = gelu(conv1d(x, self.p["conv2.weight"], self.p["conv2.bias"], 2, 1)).transpose(0, 2, 1)
        kv = []
        for i in range(self.n_enc):
            x, (k, v) = self.layer(f"encoder_layers.{i}", x, is_decoder=False)
            kv.append((k, v))
        return layer_norm(x, self.p["encoder_norm.weight"], self.p["encoder_norm.bias"]), kv

    def project_cross_kv(self, enc_hidden: np.ndarray):
        """Per decoder layer (K, V) = cross_attn_k/v(encoder states) (models.py:179-181)."""
        out = []
        for i in range(self.n_dec):
            pre = f"decoder_layers.{i}"
            out.append((self._heads(linear(enc_hidden, self.p[f"{pre}.cross_attn_k.weight"])),
                        self._heads(linear(enc_hidden, self.p[f"{pre}.cross_attn_v.weight"]))))
        return out

    def decode_step(self, ids: np.ndarray, past: Optional[List[Tuple[np.ndarray, np.ndarray]]],
                    cross: Optional[Sequence[Tuple[np.ndarray, np.ndarray]]]):
        """models.py:369-423; ids [B, S] -> logits [B, S, V], new per-layer (K, V)."""
        x = self.p["decoder_embed.weight"][np.asarray(ids)]
        new = []
        for i in range(self.n_dec):
            pk = past[i] if past is not None else None
            ck = cross[i] if cross is not None and i < len(cross) else None
            x, kv = self.layer(f"decoder_layers.{i}", x, pk, ck)
            new.append(kv)
        x = layer_norm(x, self.p["decoder_norm.weight"], self.p["decoder_norm.bias"])
        return linear(x, self.p["lm_head.weight"]), new

    def greedy(self, prompt: Sequence[int], cross: Optional[Sequence[Tuple[np.ndarray, np.ndarray]]],
               max_new_tokens: int, eos: Optional[int] = None) -> Tuple[List[int], List[np.ndarray]]:
        """Prefill the prompt, then one token per step; stops after EOS (kept) or max_new_tokens."""
        logits, past = self.decode_step(np.asarray([list(prompt)]), None, cross)
        toks, all_logits = [], []
        while True:
            last = logits[0, -1]
            all_logits.append(last)
            t = int(np.argmax(last))
            toks.append(t)
            if (eos is not None and t == eos) or len(toks) >= max_new_tokens:
                return toks, all_logits
            logits, past = self.decode_step(np.asarray([[t]]), past, cross)
