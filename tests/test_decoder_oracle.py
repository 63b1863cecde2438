"""Pin oracle/decoder.py to golden vectors written from the reference model
(tests/golden/make_golden.py). CPU only.

The reference computes in float32; the oracle in float64, so values agree to
float32 rounding (rtol/atol 2e-5 on O(1) logits) and greedy tokens agree
exactly. Planted mistakes in the oracle (wrong MLP norm, no causal mask,
tanh-approximate GELU) must break the match.
"""
import json
import os

import numpy as np
import pytest

from oracle import decoder as D

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "whisper_tiny_golden.npz")


@pytest.fixture(scope="module")
def gold():
    z = np.load(GOLDEN, allow_pickle=False)
    cfg = json.loads(bytes(z["config_json"]).decode())
    state = {k[len("param."):]: z[k] for k in z.files if k.startswith("param.")}
    return z, cfg, state


def make(cfg, state):
    return D.Model(state, cfg["num_heads"], cfg["hidden_dim"] // cfg["num_heads"])


def enc_kv(z, n):
    return [(z[f"enc_k{l}"].astype(np.float64), z[f"enc_v{l}"].astype(np.float64)) for l in range(n)]


def test_encode_matches_reference(gold):
    z, cfg, state = gold
    m = make(cfg, state)
    hidden, kv = m.encode(z["mel"])
    np.testing.assert_allclose(hidden, z["enc_hidden"], rtol=2e-5, atol=2e-5)
    for l, (k, v) in enumerate(kv):
        np.testing.assert_allclose(k, z[f"enc_k{l}"], rtol=2e-5, atol=2e-5)
        np.testing.assert_allclose(v, z[f"enc_v{l}"], rtol=2e-5, atol=2e-5)


def test_prefill_logits_and_cache_match_reference(gold):
    z, cfg, state = gold
    m = make(cfg, state)
    logits, past = m.decode_step(np.asarray([cfg["prompt"]]), None, enc_kv(z, cfg["num_encoder_layers"]))
    np.testing.assert_allclose(logits, z["prefill_logits"], rtol=2e-5, atol=2e-5)
    for l, (k, v) in enumerate(past):
        np.testing.assert_allclose(k, z[f"prefill_k{l}"], rtol=2e-5, atol=2e-5)
        np.testing.assert_allclose(v, z[f"prefill_v{l}"], rtol=2e-5, atol=2e-5)


def test_greedy_tokens_identical_to_reference(gold):
    z, cfg, state = gold
    m = make(cfg, state)
    toks, logits = m.greedy(cfg["prompt"], enc_kv(z, cfg["num_encoder_layers"]), cfg["new_tokens"])
    assert toks == z["greedy_tokens"].tolist()
    np.testing.assert_allclose(np.stack(logits), z["greedy_logits"], rtol=2e-5, atol=2e-5)


def test_projected_cross_kv_path_matches_reference(gold):
    """decode_step(encoder_hidden_states=...) projects cross K/V with cross_attn_k/v."""
    z, cfg, state = gold
    m = make(cfg, state)
    cross = m.project_cross_kv(z["enc_hidden"].astype(np.float64))
    logits, _ = m.decode_step(np.asarray([cfg["prompt"]]), None, cross)
    np.testing.assert_allclose(logits, z["proj_logits"], rtol=2e-5, atol=2e-5)


class _NormSwap(D.Model):
    def layer(self, prefix, x, past=None, cross=None, is_decoder=True):
        p = dict(self.p)
        if cross is not None:
            self.p[f"{prefix}.norm3.weight"], self.p[f"{prefix}.norm3.bias"] = (p[f"{prefix}.norm2.weight"],
                                                                              p[f"{prefix}.norm2.bias"])
        try:
            return super().layer(prefix, x, past, cross, is_decoder)
        finally:
            self.p = p


class _NoCausal(D.Model):
    def layer(self, prefix, x, past=None, cross=None, is_decoder=True):
        return super().layer(prefix, x, past, cross, is_decoder=False)


@pytest.mark.parametrize("mutant", ["norm2_for_mlp", "no_causal_mask", "tanh_gelu"])
def test_golden_catches_planted_oracle_mistakes(gold, mutant, monkeypatch):
    z, cfg, state = gold
    hd = cfg["hidden_dim"] // cfg["num_heads"]
    if mutant == "norm2_for_mlp":
        m = _NormSwap(state, cfg["num_heads"], hd)
    elif mutant == "no_causal_mask":
        m = _NoCausal(state, cfg["num_heads"], hd)
    else:
        m = make(cfg, state)
        monkeypatch.setattr(D, "gelu", lambda x: 0.5 * x * (1 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3))))
    logits, _ = m.decode_step(np.asarray([cfg["prompt"]]), None, enc_kv(z, cfg["num_encoder_layers"]))
    assert not np.allclose(logits, z["prefill_logits"], rtol=2e-5, atol=2e-5)
