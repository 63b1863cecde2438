"""Pins oracle/cpu_path.py — the float32 torch restatement of the reference's eager CPU path that
bench.py times as the CPU baseline — against the reference's golden vectors and the float64 oracle.

- Decoder: prefill logits and K/V and the 8 greedy tokens and their logits of the reference's tiny
  Whisper-class model (tests/golden/whisper_tiny_golden.npz).
- EagerDecode: batched greedy decoding of requests with different encoder lengths (padded and
  masked, as the reference scheduler batches them) equals each request decoded alone by the
  float64 oracle.
- paged_attention_step: the new rows land in the pool bit for bit, and the output equals the
  float64 oracle's paged attention over the pool.
- TTSModel / tts_step: the reference TTS model's prefill logits and its engine's frames
  (tests/golden/tts_small_golden.npz), frame by frame through the block pool.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import cpu_path as C
from oracle import decoder as D
from oracle import paged_kv as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    z = np.load(os.path.join(GOLD, name), allow_pickle=False)
    cfg = json.loads(bytes(z["config_json"]).decode())
    state = {k[len("param."):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param.")}
    return z, cfg, state


def test_decoder_matches_reference_golden():
    z, cfg, state = load("whisper_tiny_golden.npz")
    dec = C.Decoder(state, cfg["num_heads"], cfg["hidden_dim"] // cfg["num_heads"])
    enc = [(torch.from_numpy(z[f"enc_k{l}"]), torch.from_numpy(z[f"enc_v{l}"]))
           for l in range(cfg["num_encoder_layers"])]
    with torch.no_grad():
        logits, past = dec.decode_step(torch.tensor([cfg["prompt"]]), None, enc)
        np.testing.assert_allclose(logits.numpy(), z["prefill_logits"], atol=2e-5, rtol=0)
        for l in range(cfg["num_decoder_layers"]):
            np.testing.assert_allclose(past[l][0].numpy(), z[f"prefill_k{l}"], atol=1e-5, rtol=0)
            np.testing.assert_allclose(past[l][1].numpy(), z[f"prefill_v{l}"], atol=1e-5, rtol=0)
        toks, all_logits = [], []
        for _ in range(cfg["new_tokens"]):
            all_logits.append(logits[0, -1].numpy())
            toks.append(int(logits[0, -1].argmax()))
            logits, past = dec.decode_step(torch.tensor([[toks[-1]]]), past, enc)
    assert toks == z["greedy_tokens"].tolist()
    np.testing.assert_allclose(np.stack(all_logits), z["greedy_logits"], atol=2e-5, rtol=0)


def small_model(seed=0, layers=2, heads=4, d=16, hidden=64, vocab=101):
    g = torch.Generator().manual_seed(seed)
    state = {"decoder_embed.weight": torch.randn(vocab, hidden, generator=g),
             "lm_head.weight": torch.randn(vocab, hidden, generator=g) * 0.2,
             "decoder_norm.weight": 1 + 0.1 * torch.randn(hidden, generator=g),
             "decoder_norm.bias": 0.1 * torch.randn(hidden, generator=g)}
    for i in range(layers):
        pre = f"decoder_layers.{i}."
        for n in ("self_attn_q", "self_attn_k", "self_attn_v", "cross_attn_q"):
            state[pre + n + ".weight"] = torch.randn(heads * d, hidden, generator=g) * 0.2
        for n in ("self_attn_out", "cross_attn_out"):
            state[pre + n + ".weight"] = torch.randn(hidden, heads * d, generator=g) * 0.2
        for n in ("norm1", "norm2", "norm3"):
            state[pre + n + ".weight"] = 1 + 0.1 * torch.randn(hidden, generator=g)
            state[pre + n + ".bias"] = 0.1 * torch.randn(hidden, generator=g)
        state[pre + "mlp.0.weight"] = torch.randn(4 * hidden, hidden, generator=g) * 0.2
        state[pre + "mlp.0.bias"] = 0.1 * torch.randn(4 * hidden, generator=g)
        state[pre + "mlp.2.weight"] = torch.randn(hidden, 4 * hidden, generator=g) * 0.1
        state[pre + "mlp.2.bias"] = 0.1 * torch.randn(hidden, generator=g)
    return state, heads, d


def test_eager_decode_batches_like_one_request_at_a_time():
    state, h, d = small_model()
    g = torch.Generator().manual_seed(1)
    lens = [37, 90, 64]
    cross = [[(torch.randn(1, h, t, d, generator=g), torch.randn(1, h, t, d, generator=g)) for _ in range(2)]
             for t in lens]
    prompt = [5, 7, 11]
    run = C.EagerDecode(C.Decoder(state, h, d), cross, block_size=8)
    with torch.no_grad():
        toks, steps, _ = run.run(prompt, 12)
    assert steps == 11
    om = D.Model({k: v.numpy() for k, v in state.items()}, h, d)
    for r, c in enumerate(cross):
        want, _ = om.greedy(prompt, [(k.double().numpy(), v.double().numpy()) for k, v in c], 12)
        assert toks[r] == want, r


def test_paged_attention_step_matches_the_oracle():
    g = torch.Generator().manual_seed(3)
    b, h, d, bs, nb = 5, 4, 32, 16, 80
    ctx = [1, 16, 17, 100, 200]
    tables = torch.randperm(nb, generator=g)[: b * 13].view(b, 13)
    kp, vp = torch.randn(nb, bs, h, d, generator=g), torch.randn(nb, bs, h, d, generator=g)
    q, kn, vn = (torch.randn(b, h, d, generator=g) for _ in range(3))
    out = C.paged_attention_step(q, kp, vp, tables, ctx, kn, vn, 1 / math.sqrt(d))
    for i, c in enumerate(ctx):
        blk = int(tables[i, (c - 1) // bs])
        assert torch.equal(kp[blk, (c - 1) % bs], kn[i]) and torch.equal(vp[blk, (c - 1) % bs], vn[i])
    want = O.paged_attention(q.double().numpy()[:, None], kp.double().numpy(), vp.double().numpy(), tables.numpy(),
                             ctx, 1 / math.sqrt(d))[:, 0]
    np.testing.assert_allclose(out.numpy(), want, atol=2e-6, rtol=0)


def test_tts_steps_match_reference_engine():
    z, cfg, state = load("tts_small_golden.npz")
    h = cfg["num_heads"]
    model = C.TTSModel(state, h, cfg["hidden_dim"] // h)
    bs = cfg["block_size"]
    p, f = cfg["prompt_len"], cfg["frames"]
    for r in range(cfg["requests"]):
        pools = [(torch.zeros(8, bs, h, cfg["hidden_dim"] // h), torch.zeros(8, bs, h, cfg["hidden_dim"] // h))
                 for _ in range(cfg["num_layers"])]
        table = list(range(-(-(p + f) // bs)))
        with torch.no_grad():
            logits, kv = model.forward(torch.from_numpy(z["prompts"][r])[None])
            np.testing.assert_allclose(logits.numpy(), z[f"prefill_logits{r}"], atol=2e-5, rtol=0)
            for (kpl, vpl), (k, v) in zip(pools, kv):  # prefill write (tts_engine.py:114-128)
                for pos in range(p):
                    kpl[table[pos // bs], pos % bs] = k[0, :, pos]
                    vpl[table[pos // bs], pos % bs] = v[0, :, pos]
            frames = [logits[0, -1].argmax(-1)]
            for s in range(1, f):
                frames.append(C.tts_step(model, pools, table, p + s - 1, frames[-1][None, None]))
        assert np.array_equal(torch.stack(frames).numpy(), z[f"engine_frames{r}"]), r
