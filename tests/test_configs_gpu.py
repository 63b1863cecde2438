"""Serving scenarios of the benchmark configurations, end to end on the GPU.

  C3  Whisper-base-shaped decoder (6 layers, d_model 512, 8 heads x 64, fp16) at batch 32: 32 slots
      serving 64 requests whose encoder outputs have valid lengths U[500, 1500] (the explicit
      cross-attention mask of the reference, expressed as per-request lengths), 224 greedy tokens
      each, continuous batching with graph-slot reuse (the second 32 requests take the slots the
      first 32 free). Graph decode must give the eager decode's tokens.
  C4  Whisper-small-shaped decoder (12 layers, d_model 768, 12 heads x 64, bf16), 64 graph slots with
      batch buckets 1/8/16/32/64, Poisson arrivals (lambda = 4 req/s on a simulated clock) of 200
      requests with output lengths U[16, 448], readback every 4 steps.
  C5  Whisper-large-v3-shaped decoder (all 32 layers, d_model 1280, 20 heads x 64, vocab 51866,
      bf16), 128 graph slots, a burst of 256 requests with 1500 encoder positions and 448 tokens
      each, and a decoder pool smaller than the burst needs, so admission waits for blocks and
      blocks are recycled.

Every scenario also holds four of its requests' greedy tokens to the float64 oracle on the same
(rounded) weights and encoder K/V, teacher-forced along the GPU's tokens (precision_check.py): the
GPU logits stay within E = 8 u sqrt(L) rms(logits) of the oracle's (u the dtype's unit roundoff, L
the layers), and each GPU token is the oracle's argmax or, at a near-tie, within 2E of it. C3 is
compared over all 224 tokens, C4 and C5 over their first 32.

Random-init weights N(0, 0.02); EOS disabled so every request runs to its length.
Mirrors the reference's scenario drivers (scripts/evaluate_real_speech.py:774-779 arrivals,
phase_aware_scheduler.py:654-656 up-front graph blocks) and its sequential-vs-batched token check
(test_speech_engine.py:237-298).
"""
import numpy as np
import pytest
import torch

from speech_serving.block_manager import BlockManager
from speech_serving.dual_cache_manager import DualCacheManager
from speech_serving.encoder_block_manager import EncoderBlockManager
from speech_serving.memory_guard import MemoryGuard
from speech_serving.models import WhisperClassSpeechEncoderDecoderModel
from speech_serving.phase_aware_scheduler import PhaseAwareSpeechScheduler, RequestPhase

import precision_check as P

pytestmark = pytest.mark.gpu

PROMPT = [50258, 50259, 50359, 50363]
# Admission backpressure off: every submitted request queues and waits for a slot and blocks.
QUEUE_ALL = MemoryGuard(high_water_mark_pct=1e9)


def model(cuda, layers, d_model, heads, vocab, dtype, seed):
    m = WhisperClassSpeechEncoderDecoderModel(1, layers, heads, d_model, 80, vocab, head_dim=64)
    return m.init_normal_(0.02, seed=seed, draw_device=str(cuda)).to(cuda, dtype).eval()


def oracle_check(m, kvs, paths, steps):
    """Four requests' tokens (paths) against the float64 oracle on the same weights and encoder K/V,
    with the GPU's eager logits along the same tokens; returns the comparison's statistics."""
    om = P.oracle_of(m)
    cross = [[(k.double().cpu().numpy(), v.double().cpu().numpy()) for k, v in kv] for kv in kvs]
    want = P.oracle_logits_along(om, PROMPT, cross, paths, steps)
    del om, cross
    got = P.gpu_logits_along(m, PROMPT, kvs, paths, steps)
    stats = P.check_tokens(m.dtype, m.num_decoder_layers, want, paths, gpu_logits=got)
    print("float64 oracle comparison:", stats)
    return stats


def managers(m, cuda, dtype, dec_blocks, enc_blocks=16):
    enc = EncoderBlockManager(m.num_encoder_layers, m.num_heads, m.head_dim, 16, enc_blocks, dtype=dtype,
                              device=str(cuda))
    dec = BlockManager(m.num_decoder_layers, m.num_heads, m.head_dim, 16, dec_blocks, dtype=dtype, device=str(cuda))
    return enc, dec


def encoder_kv(m, cuda, t, seed):
    gen = torch.Generator().manual_seed(seed)
    states = torch.randn(1, t, m.hidden_dim, generator=gen).to(cuda, m.decoder_norm.weight.dtype)
    with torch.no_grad():
        return m.project_cross_kv(states)


def test_c3_base_variable_encoder_lengths_graph_matches_eager(cuda):
    dt = torch.float16
    m = model(cuda, 6, 512, 8, 51865, dt, seed=3)
    lengths = np.random.default_rng(3).integers(500, 1501, size=64).tolist()
    kvs = [encoder_kv(m, cuda, t, 100 + i) for i, t in enumerate(lengths)]
    results = {}
    for mode in ("eager", "graph"):
        enc, dec = managers(m, cuda, dt, dec_blocks=512)
        kw = dict(graph_decode=True, graph_readback_k=4, graph_direct_encoder_kv=True, graph_max_enc_len=1500) \
            if mode == "graph" else {}
        s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), QUEUE_ALL, max_batch_size=32,
                                      device=str(cuda), eos_token_id=-1, **kw)
        for kv in kvs:
            s.submit_encoded(kv, prompt_token_ids=torch.tensor([PROMPT]), max_new_tokens=224)
        done = sorted(s.run_until_done(), key=lambda r: r.id)
        assert len(done) == 64 and all(r.phase == RequestPhase.COMPLETED for r in done)
        assert s.peak_in_flight_requests == 32
        assert all(len(r.generated_tokens) == 224 for r in done)
        assert [r.encoder_seq_len for r in done] == lengths
        assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0
        if mode == "graph":
            assert any(r.graph_slot_reused for r in done)
            assert s.graph_buffers.active_slot_count() == 0
        results[mode] = [r.generated_tokens for r in done]
    assert results["graph"] == results["eager"]
    # the shortest and the longest encoder outputs, and the first requests
    pick = list(dict.fromkeys([int(np.argmin(lengths)), int(np.argmax(lengths)), 0, 1, 2]))[:4]
    oracle_check(m, [kvs[i] for i in pick], [results["graph"][i] for i in pick], 224)


def test_c4_small_poisson_arrivals_with_buckets(cuda):
    dt = torch.bfloat16
    m = model(cuda, 12, 768, 12, 51865, dt, seed=4)
    rng = np.random.default_rng(4)
    n = 200
    arrivals = np.cumsum(rng.exponential(1 / 4.0, size=n))
    arrivals -= arrivals[0]  # first arrival at t = 0
    out_lens = rng.integers(16, 449, size=n).tolist()
    kvs = [encoder_kv(m, cuda, 1500, 400 + i) for i in range(8)]
    enc, dec = managers(m, cuda, dt, dec_blocks=64 * 29 + 64)
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), QUEUE_ALL, max_batch_size=64,
                                  device=str(cuda), eos_token_id=-1, graph_decode=True, graph_readback_k=4,
                                  graph_direct_encoder_kv=True, graph_max_enc_len=1500)
    clock, step_s, nxt, buckets = 0.0, 0.05, 0, set()
    finished = []
    while len(finished) < n:
        while nxt < n and arrivals[nxt] <= clock:
            s.submit_encoded(kvs[nxt % 8], prompt_token_ids=torch.tensor([PROMPT]), max_new_tokens=out_lens[nxt],
                             arrival_time=float(arrivals[nxt]))
            nxt += 1
        s.step()
        if s.active_decode:
            buckets.add(s.graph_buffers.pick_bucket(len(s.active_decode)))
        finished = list(s.completed)
        clock += step_s
        assert clock < 10_000, "scenario did not drain"
    done = sorted(finished, key=lambda r: r.id)
    assert [len(r.generated_tokens) for r in done] == out_lens
    assert all(r.phase == RequestPhase.COMPLETED for r in done)
    assert len(buckets) >= 3, buckets
    assert dec.allocated_block_count == 0 and s.graph_buffers.active_slot_count() == 0
    first = {}
    for i, r in enumerate(done):  # request i used encoder output i % 8
        if len(r.generated_tokens) >= 32 and i % 8 not in first:
            first[i % 8] = r.generated_tokens
    keys = sorted(first)[:4]
    oracle_check(m, [kvs[k] for k in keys], [first[k] for k in keys], 32)


def test_c5_large_v3_burst_exhausts_and_recycles_the_pool(cuda):
    dt = torch.bfloat16
    m = model(cuda, 32, 1280, 20, 51866, dt, seed=5)
    per_req = -(-(len(PROMPT) + 448) // 16)  # 29 blocks reserved up front per graph request
    pool = 128 * per_req + 100               # room for the 128 slots, not for the 256-request burst
    kvs = [encoder_kv(m, cuda, 1500, 500 + i) for i in range(8)]
    enc, dec = managers(m, cuda, dt, dec_blocks=pool)
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), QUEUE_ALL, max_batch_size=128,
                                  device=str(cuda), eos_token_id=-1, graph_decode=True, graph_readback_k=4,
                                  graph_direct_encoder_kv=True, graph_max_enc_len=1500)
    for i in range(256):
        s.submit_encoded(kvs[i % 8], prompt_token_ids=torch.tensor([PROMPT]), max_new_tokens=448)
    peak = 0
    while s.step():
        peak = max(peak, dec.allocated_block_count)
    done = sorted(s.completed, key=lambda r: r.id)
    assert len(done) == 256 and all(len(r.generated_tokens) == 448 for r in done)
    assert per_req * 128 <= peak <= pool  # the pool filled up and was never exceeded
    assert any(r.graph_slot_reused for r in done)
    assert dec.allocated_block_count == 0 and dec.num_free_blocks == pool
    # Requests with the same encoder output and prompt decode the same tokens whichever slot and batch they got.
    by_kv = {}
    for r in done:
        by_kv.setdefault((r.id - done[0].id) % 8, set()).add(tuple(r.generated_tokens))
    assert all(len(v) == 1 for v in by_kv.values())
    del s, enc, dec
    torch.cuda.empty_cache()
    oracle_check(m, kvs[:4], [list(next(iter(by_kv[k]))) for k in range(4)], 32)
