"""Pins oracle/tts.py: golden vectors from the reference's TTS model and engine, plus invariants.

- TTSModel.forward / generate against tests/golden/tts_small_golden.npz (written by
  tests/golden/make_tts_golden.py from the reference implementation, CPU float32):
  prefill logits and K/V, every generated frame's logits, and the reference engine's frames.
- Incremental decoding with the contiguous past equals one causal pass over the whole
  sequence (pins the causal mask and the cache concatenation independently of the golden file).
- Engine bookkeeping: completion order, LIFO block ids, the closed form for a request's
  block count after f frames, and every block returned at the end.
"""
import json
import math
import os

import numpy as np
import pytest

from oracle.tts import Engine, TTSModel

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "tts_small_golden.npz")


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN)
    cfg = json.loads(bytes(z["config_json"]).decode())
    state = {k[len("param."):]: z[k] for k in z.files if k.startswith("param.")}
    model = TTSModel(state, cfg["num_heads"], cfg["hidden_dim"] // cfg["num_heads"])
    return z, cfg, model


def test_prefill_matches_reference(golden):
    z, cfg, model = golden
    for r in range(cfg["requests"]):
        logits, kv = model.forward(z["prompts"][r][None])
        np.testing.assert_allclose(logits, z[f"prefill_logits{r}"], atol=2e-4, rtol=0)
        if r == 0:
            for l in range(cfg["num_layers"]):
                np.testing.assert_allclose(kv[l][0], z[f"prefill_k{l}"], atol=1e-5, rtol=0)
                np.testing.assert_allclose(kv[l][1], z[f"prefill_v{l}"], atol=1e-5, rtol=0)


def test_generated_frames_match_reference_engine(golden):
    z, cfg, model = golden
    for r in range(cfg["requests"]):
        frames, logits = model.generate(z["prompts"][r], cfg["frames"])
        np.testing.assert_allclose(logits, z[f"step_logits{r}"], atol=2e-4, rtol=0)
        assert np.array_equal(frames, z[f"engine_frames{r}"]), r
        assert frames.shape == (cfg["frames"], cfg["num_codebooks"])


def test_incremental_equals_one_causal_pass(golden):
    z, cfg, model = golden
    prompt = z["prompts"][1]
    frames, logits = model.generate(prompt, 6)
    whole = np.concatenate([prompt, frames[:-1]], axis=0)[None]  # every input frame at once
    full, _ = model.forward(whole)
    p = prompt.shape[0]
    np.testing.assert_allclose(full[0, p - 1:], logits, atol=1e-9, rtol=0)


def test_heads_and_embedding_reduce_to_single_codebook_lookups(golden):
    """With one nonzero codebook the embedding is that codebook's row and the heads are per-codebook GEMVs."""
    z, cfg, model = golden
    codes = np.zeros((1, 1, cfg["num_codebooks"]), dtype=np.int64)
    codes[0, 0, 2] = 5
    e = model.embed(codes)[0, 0]
    expect = model.p["embeddings.embeddings.2.weight"][5] + sum(
        model.p[f"embeddings.embeddings.{k}.weight"][0] for k in (0, 1, 3))
    np.testing.assert_allclose(e, expect, atol=1e-12)
    x = np.random.default_rng(0).standard_normal((1, 1, cfg["hidden_dim"]))
    h = model.heads(x)
    for k in range(cfg["num_codebooks"]):
        np.testing.assert_allclose(h[0, 0, k], model.p[f"heads.heads.{k}.weight"] @ x[0, 0], atol=1e-12)


def test_engine_bookkeeping(golden):
    z, cfg, _ = golden
    eng = Engine(cfg["num_blocks"], cfg["block_size"], cfg["max_batch"])
    lens = [cfg["prompt_len"]] * cfg["requests"]
    done, history, peak = eng.run(lens, [cfg["frames"]] * cfg["requests"])
    assert done == [0, 1, 2]
    assert sorted(eng.free) == list(range(cfg["num_blocks"]))
    assert z["engine_blocks"].tolist() == [0, cfg["num_blocks"]]
    bs = cfg["block_size"]
    for r, tables in history.items():
        assert len(tables) == cfg["frames"]
        for f, t in enumerate(tables, start=1):
            assert len(t) == math.ceil((cfg["prompt_len"] + f - 1) / bs), (r, f)
    assert history[0][0] == [31, 30]  # LIFO: the last free ids first
    assert peak <= cfg["max_batch"] * math.ceil((cfg["prompt_len"] + cfg["frames"] - 1) / bs)


def test_engine_immediate_completion_and_exhaustion():
    eng = Engine(4, 4, 2)
    done, history, _ = eng.run([3, 5], [1, 2])
    assert done == [0, 1]  # a one-frame request completes at admission
    assert history[0] == [[3]]
    assert sorted(eng.free) == [0, 1, 2, 3]
    with pytest.raises(IndexError):
        Engine(1, 4, 1).run([9], [2])  # needs 3 blocks, the pool holds 1
