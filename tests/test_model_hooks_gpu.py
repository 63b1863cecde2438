"""The scheduler drives the model only through the reference's hooks (model.encode, model.decode_step
with the reference's keyword arguments; speech_serving/phase_aware_scheduler.py:664-670, 982-991), so
code that wraps model.decode_step sees, and can change, every eager prefill and decode step:

- the reference's test_encoder_hit_produces_identical_output (test_speech_engine.py:305-391): a wrapper
  captures encoder_past_kv_list on the miss and the hit path; the captured K/V agree (and equal the
  encoder's own K/V, the reference's synthetic model attending its encoder layers' K/V);
- the reference's test_generation_stops_on_eos_and_uses_whisper_prompt (:549-613): a wrapper forces EOS
  from the third call on; the request stops there, keeps EOS and leaks nothing;
- a model that has only the reference's hooks (no paged step) is served eagerly on K/V gathered from
  the pool (skv_gather -> decode_step -> skv_append) and decodes the reference's golden tokens, and a
  variable-length batch of such requests the one-at-a-time oracle tokens; graph decode refuses it;
- the PagedKVCache a paged decode_step returns reads back like the reference's DynamicCache.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import decoder as D
from speech_serving import native
from speech_serving.block_manager import BlockManager
from speech_serving.dual_cache_manager import DualCacheManager
from speech_serving.encoder_block_manager import EncoderBlockManager
from speech_serving.memory_guard import MemoryGuard
from speech_serving.models import PagedKVCache, WhisperClassSpeechEncoderDecoderModel
from speech_serving.phase_aware_scheduler import PhaseAwareSpeechScheduler, RequestPhase

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "whisper_tiny_golden.npz")


class HookOnlyModel:
    """A model that offers the scheduler only the reference's hooks: encode, decode_step (contiguous past
    K/V, as the reference's model; here the GPU model's own contiguous decode_step) and the attributes
    the scheduler reads. No paged step."""

    def __init__(self, m):
        self._m = m
        for a in ("num_decoder_layers", "num_encoder_layers", "num_heads", "head_dim", "hidden_dim", "vocab_size",
                  "config"):
            setattr(self, a, getattr(m, a))
        self.calls = []

    def encode(self, mel):
        return self._m.encode(mel)

    def decode_step(self, input_ids, past_key_values=None, **kwargs):
        assert not isinstance(past_key_values, PagedKVCache)
        assert "logits_to_keep" not in kwargs  # only the reference's keywords reach a hook-only model
        self.calls.append((tuple(input_ids.shape), past_key_values is None))
        return self._m.decode_step(input_ids, past_key_values=past_key_values, **kwargs)


def tiny(cuda, vocab, seed, dtype=torch.float32):
    torch.manual_seed(seed)
    return WhisperClassSpeechEncoderDecoderModel(num_encoder_layers=2, num_decoder_layers=2, num_heads=4,
                                                 hidden_dim=64, mel_dim=80, vocab_size=vocab).to(cuda, dtype).eval()


def pools(cuda, layers=2, heads=4, head_dim=16, bs=8, blocks=64, dtype=torch.float32):
    enc = EncoderBlockManager(layers, heads, head_dim, bs, blocks, dtype=dtype, device=str(cuda))
    dec = BlockManager(layers, heads, head_dim, bs, blocks, dtype=dtype, device=str(cuda))
    return enc, dec


@pytest.mark.parametrize("retain", [False, True])
def test_decode_step_wrapper_sees_encoder_kv_on_miss_and_hit(cuda, retain):
    m = tiny(cuda, 256, 7)
    enc_bm, dec_bm = pools(cuda)
    s = PhaseAwareSpeechScheduler(model=m, dual_cache_manager=DualCacheManager(enc_bm, dec_bm),
                                  memory_guard=MemoryGuard(), max_batch_size=2, device=str(cuda),
                                  retain_encoder_cache=retain)
    mel = torch.randn(80, 32, generator=torch.Generator().manual_seed(7)).to(cuda)

    gathered, calls = [], []
    original = m.decode_step

    def hooked_decode(input_ids, past_key_values=None, encoder_past_kv_list=None, **kwargs):
        calls.append(tuple(input_ids.shape))
        if encoder_past_kv_list is not None:
            gathered.append([(k.clone(), v.clone()) for (k, v) in encoder_past_kv_list])
        return original(input_ids, past_key_values=past_key_values, encoder_past_kv_list=encoder_past_kv_list,
                        **kwargs)

    m.decode_step = hooked_decode
    s.submit(mel.clone(), max_new_tokens=8)
    first = s.run_until_done()
    assert len(first) == 1
    tokens_first = first[0].generated_tokens[:]
    n_first = len(gathered)
    s.completed.clear()
    s.submit(mel.clone(), max_new_tokens=8)
    second = s.run_until_done()
    assert len(second) == 1
    m.decode_step = original

    assert tokens_first == second[0].generated_tokens and len(tokens_first) == 8
    # one prefill (the 1-token default prompt) and 7 decode steps per request, every one through the
    # wrapper with the encoder K/V
    assert calls == [(1, 1)] * 16 and len(gathered) == 16 and n_first == 8
    if retain:
        assert s.encoder_calls == 1 and s.encoder_calls_skipped == 1  # the second request was a hit
    with torch.no_grad():
        _, enc_kv = m.encode(mel[None])
    t = enc_kv[0][0].shape[2]
    for i, kv in enumerate(gathered):  # miss prefill, miss decode steps, hit prefill, hit decode steps
        assert len(kv) == 2
        for l, (k, v) in enumerate(kv):
            assert tuple(k.shape) == (1, 4, t, 16) and tuple(v.shape) == (1, 4, t, 16)
            assert torch.allclose(k, gathered[0][l][0], atol=1e-5, rtol=1e-5), f"call {i} layer {l}"
            assert torch.allclose(v, gathered[0][l][1], atol=1e-5, rtol=1e-5), f"call {i} layer {l}"
            assert torch.allclose(k, enc_kv[l][0], atol=1e-5, rtol=1e-5)
            assert torch.allclose(v, enc_kv[l][1], atol=1e-5, rtol=1e-5)
    assert dec_bm.allocated_block_count == 0
    s.flush_retained_caches()
    assert enc_bm.allocated_block_count == 0


@pytest.mark.parametrize("hook_only", [False, True])
def test_decode_step_wrapper_forces_eos(cuda, hook_only):
    target_eos = 42
    m = tiny(cuda, 512, 11)
    model = HookOnlyModel(m) if hook_only else m
    enc_bm, dec_bm = pools(cuda)
    s = PhaseAwareSpeechScheduler(model=model, dual_cache_manager=DualCacheManager(enc_bm, dec_bm),
                                  memory_guard=MemoryGuard(), max_batch_size=2, device=str(cuda),
                                  eos_token_id=target_eos)
    step_counter = [0]
    real_decode = model.decode_step

    def mock_decode(*args, **kwargs):
        out = real_decode(*args, **kwargs)
        step_counter[0] += 1
        if step_counter[0] >= 3:
            out.logits[:, -1, :] = -1e4
            out.logits[:, -1, target_eos] = 1e4
        return out

    model.decode_step = mock_decode
    mel = torch.randn(80, 32, generator=torch.Generator().manual_seed(11)).to(cuda)
    prompt = torch.tensor([[1, 2, 3]], device=cuda, dtype=torch.long)
    s.submit(mel, prompt_token_ids=prompt, max_new_tokens=50, eos_token_id=target_eos)
    completed = s.run_until_done()
    model.decode_step = real_decode
    assert len(completed) == 1
    req = completed[0]
    assert req.done and req.phase == RequestPhase.COMPLETED
    assert req.generated_count == 3 < 50
    assert req.generated_tokens[-1] == target_eos and target_eos not in req.generated_tokens[:-1]
    assert enc_bm.allocated_block_count == 0 and dec_bm.allocated_block_count == 0


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN, allow_pickle=False)
    cfg = json.loads(bytes(z["config_json"]).decode())
    state = {k[len("param."):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param.")}
    return z, cfg, state


def test_hook_only_model_decodes_the_golden_tokens(golden, cuda):
    z, cfg, state = golden
    m = WhisperClassSpeechEncoderDecoderModel(cfg["num_encoder_layers"], cfg["num_decoder_layers"], cfg["num_heads"],
                                              cfg["hidden_dim"], cfg["mel_dim"], cfg["vocab_size"])
    m.load_state_dict(state)
    model = HookOnlyModel(m.to(cuda).eval())
    enc = EncoderBlockManager(m.num_encoder_layers, m.num_heads, m.head_dim, 16, 128, dtype=torch.float32,
                              device=str(cuda))
    dec = BlockManager(m.num_decoder_layers, m.num_heads, m.head_dim, 16, 128, dtype=torch.float32, device=str(cuda))
    s = PhaseAwareSpeechScheduler(model, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda))
    s.submit(torch.from_numpy(z["mel"][0]).to(cuda), prompt_token_ids=torch.tensor([cfg["prompt"]]),
             max_new_tokens=cfg["new_tokens"])
    done = s.run_until_done()
    assert [r.generated_tokens for r in done] == [z["greedy_tokens"].tolist()]
    # one prefill (no past) and new_tokens - 1 decode steps on gathered K/V
    assert model.calls == [((1, len(cfg["prompt"])), True)] + [((1, 1), False)] * (cfg["new_tokens"] - 1)
    assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0


def test_hook_only_variable_length_batch_matches_sequential_oracle(cuda):
    """Four requests with different encoder and prompt lengths decode as one batch of a hook-only model
    (ragged self-attention and encoder masks, K/V gathered and appended every step) and give each
    request's one-at-a-time oracle tokens; mid-run completions (shorter max_new_tokens) compact the batch."""
    m = tiny(cuda, 256, 999)
    model = HookOnlyModel(m)
    gen = torch.Generator().manual_seed(999)
    lengths = [40, 100, 160, 200]
    prompts = [[1], [1, 2], [4, 2, 3], [5]]
    news = [20, 9, 20, 14]
    mels = [torch.randn(80, n, generator=gen) for n in lengths]
    om = D.Model({k: v.detach().float().cpu().numpy() for k, v in m.state_dict().items()}, m.num_heads, m.head_dim)
    want = []
    for mel, pr, n in zip(mels, prompts, news):
        _, kv = om.encode(mel[None].numpy())
        want.append(om.greedy(pr, kv, n)[0])
    enc, dec = pools(cuda)
    s = PhaseAwareSpeechScheduler(model, DualCacheManager(enc, dec), MemoryGuard(), max_batch_size=4,
                                  device=str(cuda))
    for mel, pr, n in zip(mels, prompts, news):
        s.submit(mel.to(cuda), prompt_token_ids=torch.tensor([pr]), max_new_tokens=n)
    got = [r.generated_tokens for r in sorted(s.run_until_done(), key=lambda r: r.id)]
    assert got == want
    assert any(shape[0] == 4 for shape, _ in model.calls)  # the four decoded as one batch
    assert enc.allocated_block_count == 0 and dec.allocated_block_count == 0


def test_graph_decode_refuses_a_hook_only_model(cuda):
    model = HookOnlyModel(tiny(cuda, 256, 1))
    enc, dec = pools(cuda)
    with pytest.raises(TypeError, match="graph_decode=False"):
        PhaseAwareSpeechScheduler(model, DualCacheManager(enc, dec), max_batch_size=2, device=str(cuda),
                                  graph_decode=True)


def test_paged_cache_reads_back_like_the_reference_cache(cuda):
    """After a paged prefill and two paged decode steps, the PagedKVCache the last decode_step returned
    gathers, layer by layer, the K/V the contiguous decode_step accumulates for the same tokens, and the
    logits agree."""
    m = tiny(cuda, 256, 5)
    _, dec = pools(cuda)
    table = [dec.allocate_block() for _ in range(2)]
    tables = torch.tensor([table], dtype=torch.int32, device=cuda)
    gen = torch.Generator().manual_seed(5)
    enc_kv = [(torch.randn(1, 4, 30, 16, generator=gen).to(cuda), torch.randn(1, 4, 30, 16, generator=gen).to(cuda))
              for _ in range(2)]
    ids = [torch.tensor([[1, 2, 3]], device=cuda), torch.tensor([[7]], device=cuda), torch.tensor([[9]], device=cuda)]
    past, n = None, 0
    with torch.no_grad():
        for x in ids:
            n += x.shape[1]
            ctx = torch.tensor([n], dtype=torch.int32, device=cuda)
            paged = m.decode_step(x, PagedKVCache(dec.key_pool, dec.value_pool, tables, ctx, n), enc_kv,
                                  use_cache=True)
            ref = m.decode_step(x, past, enc_kv, use_cache=True)
            past = ref.past_key_values
            np.testing.assert_allclose(paged.logits.cpu().numpy(), ref.logits.cpu().numpy(), rtol=1e-4, atol=1e-4)
    assert isinstance(paged.past_key_values, PagedKVCache) and len(paged.past_key_values.layers) == 2
    for l in range(2):
        np.testing.assert_allclose(paged.past_key_values.layers[l].keys.cpu().numpy(),
                                   past.layers[l].keys.cpu().numpy(), rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(paged.past_key_values.layers[l].values.cpu().numpy(),
                                   past.layers[l].values.cpu().numpy(), rtol=1e-5, atol=1e-5)
    dec.free_blocks(table)
