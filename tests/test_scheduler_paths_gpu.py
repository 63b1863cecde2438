"""Scheduler paths beside the plain decode, mirroring the reference's engine tests
(test_speech_engine.py:305-547 encoder-cache hit, :549-613 EOS with the Whisper prompt,
:670-780 cross-K/V flag parity and leaks): whatever path a request takes, its greedy tokens are
the same and every block is returned."""
import pytest
import torch

from speech_serving.block_manager import BlockManager
from speech_serving.dual_cache_manager import DualCacheManager
from speech_serving.encoder_block_manager import EncoderBlockManager
from speech_serving.memory_guard import MemoryGuard
from speech_serving.models import WhisperClassSpeechEncoderDecoderModel
from speech_serving.phase_aware_scheduler import PhaseAwareSpeechScheduler, RequestPhase

pytestmark = pytest.mark.gpu


def tiny(cuda, vocab=256, seed=7):
    torch.manual_seed(seed)
    return WhisperClassSpeechEncoderDecoderModel(num_encoder_layers=2, num_decoder_layers=2, num_heads=4,
                                                 hidden_dim=64, mel_dim=80, vocab_size=vocab).to(cuda).eval()


def scheduler(m, cuda, **kw):
    enc = EncoderBlockManager(2, 4, 16, 8, 64, dtype=torch.float32, device=str(cuda))
    dec = BlockManager(2, 4, 16, 8, 64, dtype=torch.float32, device=str(cuda))
    return PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), MemoryGuard(), device=str(cuda), **kw), enc, dec


def counting_encode(m):
    calls = [0]
    real = m.encode

    def enc(*a, **k):
        calls[0] += 1
        return real(*a, **k)

    m.encode = enc
    return calls


def test_encoder_cache_hit_gives_identical_tokens_without_encoding(cuda):
    m = tiny(cuda)
    calls = counting_encode(m)
    s, enc, dec = scheduler(m, cuda, max_batch_size=2, retain_encoder_cache=True)
    mel = torch.randn(80, 32, generator=torch.Generator().manual_seed(1)).to(cuda)
    s.submit(mel.clone(), max_new_tokens=8)
    first = s.run_until_done()[0].generated_tokens[:]
    s.completed.clear()
    s.submit(mel.clone(), max_new_tokens=8)  # sequential duplicate: hit
    second = s.run_until_done()[0].generated_tokens[:]
    assert first == second and len(first) == 8
    assert calls[0] == 1 and s.encoder_calls_skipped == 1
    assert dec.allocated_block_count == 0
    s.flush_retained_caches()
    assert enc.allocated_block_count == 0


def test_concurrent_duplicates_encode_once_and_agree(cuda):
    """Both copies are admitted in one sweep. Encoding is synchronous here, so the first copy's cache
    entry exists when the second is admitted and the second hits it (the reference encodes both,
    test_speech_engine.py:400-420); they share one batched prefill and decode alike."""
    m = tiny(cuda)
    calls = counting_encode(m)
    s, enc, dec = scheduler(m, cuda, max_batch_size=2, retain_encoder_cache=True)
    mel = torch.randn(80, 40, generator=torch.Generator().manual_seed(2)).to(cuda)
    s.submit(mel.clone(), max_new_tokens=6)
    s.submit(mel.clone(), max_new_tokens=6)
    done = s.run_until_done()
    assert calls[0] == 1 and s.encoder_calls_skipped == 1
    assert done[0].generated_tokens == done[1].generated_tokens and len(done[0].generated_tokens) == 6
    s.flush_retained_caches()
    assert enc.allocated_block_count == 0 and dec.allocated_block_count == 0


@pytest.mark.parametrize("flags", [dict(cache_cross_kv=True), dict(avoid_redundant_cross_kv=True),
                                   dict(no_sync_decode=True), dict(batch_encoder=True)])
def test_cross_kv_and_sampling_flags_do_not_change_tokens(cuda, flags):
    m = tiny(cuda, vocab=100, seed=42)
    gen = torch.Generator().manual_seed(42)
    mels = [torch.randn(80, 120 + 40 * i, generator=gen).to(cuda) for i in range(3)]
    prompt = torch.tensor([[1, 2, 3]])
    out = []
    for kw in ({}, flags):
        s, enc, dec = scheduler(m, cuda, max_batch_size=2, **kw)
        for mel in mels:
            s.submit(mel, prompt_token_ids=prompt, max_new_tokens=8)
        out.append([r.generated_tokens for r in sorted(s.run_until_done(), key=lambda r: r.id)])
        assert enc.allocated_block_count == 0 and dec.allocated_block_count == 0
    assert out[0] == out[1]


def test_generation_stops_on_eos_with_a_task_prompt(cuda):
    """EOS forced from the third model.decode_step call on (the prefill, then decode steps), by wrapping
    decode_step as the reference's test does: the request ends at EOS, well before max_new_tokens, keeps
    EOS as its last token (eager decode) and frees its blocks."""
    eos = 42
    m = tiny(cuda, vocab=512)
    s, enc, dec = scheduler(m, cuda, max_batch_size=2, eos_token_id=eos)
    real = m.decode_step
    n = [0]

    def forced(*a, **k):
        out = real(*a, **k)
        n[0] += 1
        if n[0] >= 3:
            out.logits[:, -1, :] = -1e4
            out.logits[:, -1, eos] = 1e4
        return out

    m.decode_step = forced
    s.submit(torch.randn(80, 32).to(cuda), prompt_token_ids=torch.tensor([[1, 2, 3]]), max_new_tokens=50)
    (r,) = s.run_until_done()
    assert r.phase == RequestPhase.COMPLETED
    assert r.generated_tokens[-1] == eos and len(r.generated_tokens) == 3 and eos not in r.generated_tokens[:-1]
    assert enc.allocated_block_count == 0 and dec.allocated_block_count == 0


def test_a_block_starved_request_fails_alone(cuda):
    """Eager decode with a decoder pool one block short: at the block boundary the first request
    takes the last free block and the second cannot get one. Only the second fails (its blocks
    go back to the pool); the first decodes on, with the tokens it has when it runs alone."""
    m = tiny(cuda)
    gen = torch.Generator().manual_seed(20)
    mels = [torch.randn(80, 32, generator=gen).to(cuda) for _ in range(2)]
    prompt = torch.tensor([[1, 2, 3]])
    s, _, _ = scheduler(m, cuda, max_batch_size=2)
    s.submit(mels[0], prompt_token_ids=prompt, max_new_tokens=12)
    alone = s.run_until_done()[0].generated_tokens[:]

    enc = EncoderBlockManager(2, 4, 16, 8, 64, dtype=torch.float32, device=str(cuda))
    dec = BlockManager(2, 4, 16, 8, 3, dtype=torch.float32, device=str(cuda))  # 2 prompts + 1 spare
    # admission backpressure off: both requests are admitted into the short pool
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), MemoryGuard(high_water_mark_pct=1e9),
                                  device=str(cuda), max_batch_size=2)
    ids = [s.submit(mel, prompt_token_ids=prompt, max_new_tokens=12) for mel in mels]
    done = {r.id: r for r in s.run_until_done()}
    assert done[ids[0]].phase == RequestPhase.COMPLETED and done[ids[0]].generated_tokens == alone
    assert done[ids[1]].phase == RequestPhase.FAILED
    assert 0 < len(done[ids[1]].generated_tokens) < 12
    assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0
