"""End-to-end decode on the GPU: model, paged pool, scheduler, graph slots.

Parity bars (greedy decoding, float32 weights):
  * token ids identical to the reference's golden vectors / the numpy oracle;
  * logits within 1e-4 (float32 GPU math vs the reference's float32 CPU math);
  * eager paged decode == graph decode token for token;
  * zero leaked blocks and slots after completion or failure.
Mirrors the reference tests test_variable_length_batch_cross_attention_correctness,
test_graph_decode_parity, test_graph_decode_eos_handling,
test_graph_decode_slots_reused_different_lengths (test_speech_engine.py).
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
from speech_serving.models import CrossKV, PagedKV, WhisperClassSpeechEncoderDecoderModel
from speech_serving.phase_aware_scheduler import PhaseAwareSpeechScheduler, RequestPhase

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "whisper_tiny_golden.npz")


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN, allow_pickle=False)
    cfg = json.loads(bytes(z["config_json"]).decode())
    state = {k[len("param."):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param.")}
    return z, cfg, state


def golden_model(golden, cuda, dtype=torch.float32):
    z, cfg, state = golden
    m = WhisperClassSpeechEncoderDecoderModel(cfg["num_encoder_layers"], cfg["num_decoder_layers"], cfg["num_heads"],
                                              cfg["hidden_dim"], cfg["mel_dim"], cfg["vocab_size"])
    m.load_state_dict(state)
    return m.to(cuda, dtype).eval()


def pools(model, cuda, dtype=torch.float32, enc_blocks=128, dec_blocks=128, bs=16):
    enc = EncoderBlockManager(model.num_encoder_layers, model.num_heads, model.head_dim, bs, enc_blocks, dtype=dtype,
                              device=str(cuda))
    dec = BlockManager(model.num_decoder_layers, model.num_heads, model.head_dim, bs, dec_blocks, dtype=dtype,
                       device=str(cuda))
    return enc, dec


def close(got, want, tol=1e-4):
    g = got.detach().float().cpu().numpy()
    np.testing.assert_allclose(g, want, rtol=tol, atol=tol)


# ---------------------------------------------------------------- golden parity
def test_encode_matches_reference_golden(golden, cuda):
    z, cfg, _ = golden
    m = golden_model(golden, cuda)
    with torch.no_grad():
        hidden, kv = m.encode(torch.from_numpy(z["mel"]).to(cuda))
    close(hidden, z["enc_hidden"])
    for l, (k, v) in enumerate(kv):
        close(k, z[f"enc_k{l}"])
        close(v, z[f"enc_v{l}"])


def test_contiguous_decode_step_matches_reference_golden(golden, cuda):
    z, cfg, _ = golden
    m = golden_model(golden, cuda)
    enc = [(torch.from_numpy(z[f"enc_k{l}"]).to(cuda), torch.from_numpy(z[f"enc_v{l}"]).to(cuda))
           for l in range(cfg["num_encoder_layers"])]
    with torch.no_grad():
        out = m.decode_step(torch.tensor([cfg["prompt"]], device=cuda), None, enc)
        close(out.logits, z["prefill_logits"])
        for l in range(cfg["num_decoder_layers"]):
            close(out.past_key_values.layers[l].keys, z[f"prefill_k{l}"])
        toks = []
        for _ in range(cfg["new_tokens"]):
            t = int(out.logits[0, -1].argmax())
            toks.append(t)
            out = m.decode_step(torch.tensor([[t]], device=cuda), out.past_key_values, enc)
    assert toks == z["greedy_tokens"].tolist()
    hid = torch.from_numpy(z["enc_hidden"]).to(cuda)
    with torch.no_grad():
        proj = m.decode_step(torch.tensor([cfg["prompt"]], device=cuda), None, None, encoder_hidden_states=hid)
    close(proj.logits, z["proj_logits"])


def test_paged_decode_matches_reference_golden(golden, cuda):
    """Prefill (causal, fused append of 3 prompt tokens) + 7 single-token steps through the pool."""
    z, cfg, _ = golden
    m = golden_model(golden, cuda)
    _, dec = pools(m, cuda)
    table = [dec.allocate_block() for _ in range(2)]
    tables = torch.tensor([table], dtype=torch.int32, device=cuda)
    enc = [(torch.from_numpy(z[f"enc_k{l}"]).to(cuda), torch.from_numpy(z[f"enc_v{l}"]).to(cuda))
           for l in range(cfg["num_encoder_layers"])]
    t_enc = enc[0][0].shape[2]
    cross = CrossKV([k for k, _ in enc], [v for _, v in enc], torch.tensor([t_enc], dtype=torch.int32, device=cuda),
                    t_enc)
    p = len(cfg["prompt"])
    toks, logits_all = [], []
    with torch.no_grad():
        ids = torch.tensor([cfg["prompt"]], device=cuda)
        for step in range(cfg["new_tokens"]):
            n = p + step
            kv = PagedKV(dec.key_pool, dec.value_pool, tables, torch.tensor([n], dtype=torch.int32, device=cuda), n)
            logits = m.decode_step_paged(ids, kv, cross)
            logits_all.append(logits[0].float().cpu().numpy())
            t = int(native.argmax(logits).item())
            toks.append(t)
            ids = torch.tensor([[t]], device=cuda)
    assert toks == z["greedy_tokens"].tolist()
    np.testing.assert_allclose(np.stack(logits_all), z["greedy_logits"], rtol=1e-4, atol=1e-4)
    # the pool holds exactly the reference's prefill K/V at positions 0..2
    kg, vg = dec.gather(0, tables, torch.tensor([p], dtype=torch.int32, device=cuda), p)
    close(kg, z["prefill_k0"])
    close(vg, z["prefill_v0"])


@pytest.mark.parametrize("mode", ["eager", "graph_k1", "graph_k4"])
def test_scheduler_matches_reference_golden(golden, cuda, mode):
    z, cfg, _ = golden
    m = golden_model(golden, cuda)
    enc, dec = pools(m, cuda)
    kw = {}
    if mode != "eager":
        kw = dict(graph_decode=True, graph_readback_k=1 if mode == "graph_k1" else 4, graph_direct_encoder_kv=True)
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda), **kw)
    s.submit(torch.from_numpy(z["mel"][0]).to(cuda), prompt_token_ids=torch.tensor([cfg["prompt"]]),
             max_new_tokens=cfg["new_tokens"])
    done = s.run_until_done()
    assert [r.generated_tokens for r in done] == [z["greedy_tokens"].tolist()]
    assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0
    if mode != "eager":
        assert s.graph_buffers.cross_cache is None and s.graph_buffers.g_cross_kv is not None
        assert s.graph_buffers.active_slot_count() == 0


# ---------------------------------------------------------------- reference-style engine tests
def random_model(cuda, seed, dtype=torch.float32, **kw):
    torch.manual_seed(seed)
    cfg = dict(num_encoder_layers=2, num_decoder_layers=2, num_heads=4, hidden_dim=64, mel_dim=80, vocab_size=256)
    cfg.update(kw)
    return WhisperClassSpeechEncoderDecoderModel(**cfg).to(cuda, dtype).eval()


def oracle_of(model):
    return D.Model({k: v.detach().float().cpu().numpy() for k, v in model.state_dict().items()}, model.num_heads,
                   model.head_dim)


def test_variable_length_batch_matches_sequential_oracle(cuda):
    """Mixed encoder lengths batched together decode exactly like one-at-a-time decoding
    (reference test_speech_engine.py:237-298), checked against the numpy oracle."""
    m = random_model(cuda, 999)
    gen = torch.Generator().manual_seed(999)
    lengths = [40, 100, 160, 200]
    mels = [torch.randn(80, n, generator=gen) for n in lengths]
    om = oracle_of(m)
    want = []
    for mel in mels:
        _, kv = om.encode(mel[None].numpy())
        toks, _ = om.greedy([1], kv, 20)
        want.append(toks)
    enc, dec = pools(m, cuda, bs=8)
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), MemoryGuard(), max_batch_size=4, device=str(cuda))
    for mel in mels:
        s.submit(mel.to(cuda), max_new_tokens=20)
    got = [r.generated_tokens for r in sorted(s.run_until_done(), key=lambda r: r.id)]
    assert got == want
    assert enc.allocated_block_count == 0 and dec.allocated_block_count == 0


@pytest.mark.parametrize("mode", ["eager", "graph"])
def test_batched_prefill_mixed_prompts_matches_oracle(cuda, mode):
    """Requests admitted in one step prefill as one batch per prompt length (here three groups, interleaved
    in submission order); each request's tokens equal its own one-at-a-time oracle decode."""
    m = random_model(cuda, 4242)
    gen = torch.Generator().manual_seed(4242)
    prompts = [[1, 2, 3], [5], [7, 8, 3, 2], [9, 4, 1], [6], [2, 2, 3, 3]]
    mels = [torch.randn(80, 60 + 24 * i, generator=gen) for i in range(len(prompts))]
    om = oracle_of(m)
    want = []
    for mel, pr in zip(mels, prompts):
        _, kv = om.encode(mel[None].numpy())
        want.append(om.greedy(pr, kv, 12)[0])
    enc, dec = pools(m, cuda, bs=8)
    kw = dict(graph_decode=True, graph_readback_k=4, graph_direct_encoder_kv=True) if mode == "graph" else {}
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), MemoryGuard(), max_batch_size=8,
                                  device=str(cuda), **kw)
    for mel, pr in zip(mels, prompts):
        s.submit(mel.to(cuda), prompt_token_ids=torch.tensor([pr]), max_new_tokens=12)
    s.step()  # one step admits and prefills all six
    assert len(s.active_decode) == len(prompts) and not s.active_encode and not s.queue
    got = [r.generated_tokens for r in sorted(s.run_until_done(), key=lambda r: r.id)]
    assert got == want
    assert enc.allocated_block_count == 0 and dec.allocated_block_count == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_graph_decode_matches_eager(cuda, dtype):
    m = random_model(cuda, 42, dtype, vocab_size=100)
    gen = torch.Generator().manual_seed(42)
    mels = [torch.randn(80, 200 + 30 * i, generator=gen).to(cuda, dtype) for i in range(3)]
    prompt = torch.tensor([[1, 2]])
    results = {}
    for mode in ("eager", "graph"):
        enc, dec = pools(m, cuda, dtype)
        kw = dict(graph_decode=True, graph_readback_k=4, graph_direct_encoder_kv=True) if mode == "graph" else {}
        s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda), **kw)
        for mel in mels:
            s.submit(mel, prompt_token_ids=prompt, max_new_tokens=10)
        results[mode] = [r.generated_tokens for r in sorted(s.run_until_done(), key=lambda r: r.id)]
        assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0
    assert results["eager"] == results["graph"]


def test_graphs_survive_workspace_growth(cuda):
    """After the buckets are captured, an eager call grows the device's attention workspace (which
    drops the old buffer) and fresh allocations follow: the graphs still decode the eager tokens and
    write nothing into memory handed out after the growth."""
    dtype = torch.float16
    m = random_model(cuda, 42, dtype, vocab_size=100)
    gen = torch.Generator().manual_seed(43)
    mels = [torch.randn(80, 200 + 30 * i, generator=gen).to(cuda, dtype) for i in range(3)]
    prompt = torch.tensor([[1, 2]])
    results, junk = {}, []
    for mode in ("eager", "graph"):
        enc, dec = pools(m, cuda, dtype)
        kw = dict(graph_decode=True, graph_readback_k=4, graph_direct_encoder_kv=True) if mode == "graph" else {}
        s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda), **kw)
        for mel in mels:
            s.submit(mel, prompt_token_ids=prompt, max_new_tokens=10)
        s.step()
        if mode == "graph":
            assert s.graph_buffers is not None and s.graph_buffers.graphs
            ws = native.reserve_workspace(0, cuda)
            native.reserve_workspace(ws.numel() * 4, cuda)
            for _ in range(8):
                junk.append(torch.full((ws.numel() // 4,), 7, dtype=torch.int32, device=cuda))
        results[mode] = [r.generated_tokens for r in sorted(s.run_until_done(), key=lambda r: r.id)]
    assert results["eager"] == results["graph"]
    assert junk and all(bool((t == 7).all()) for t in junk)


def test_graph_eos_is_trimmed_eager_keeps_it(cuda):
    """Graph decode drops EOS and later tokens; eager keeps EOS as the last token
    (reference test_speech_engine.py:893-933 vs :549-613)."""
    m = random_model(cuda, 303, vocab_size=100)
    mel = torch.randn(80, 200, generator=torch.Generator().manual_seed(303)).to(cuda)
    prompt = torch.tensor([[1, 2]])

    def run(graph, eos):
        enc, dec = pools(m, cuda)
        kw = dict(graph_decode=True, graph_readback_k=4) if graph else {}
        s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda), **kw)
        s.submit(mel, prompt_token_ids=prompt, max_new_tokens=10, eos_token_id=eos)
        toks = s.run_until_done()[0].generated_tokens
        assert dec.allocated_block_count == 0
        return toks

    base = run(False, None)
    eos = base[2]
    if eos in base[:2]:
        pytest.skip("seeded model repeats the chosen EOS token early")
    g = run(True, eos)
    e = run(False, eos)
    assert g == base[:2] and eos not in g
    assert e == base[:3] and e[-1] == eos


def test_on_device_eos_retires_slots_inside_a_long_readback_window(cuda):
    """With readback every 16 steps, a request that emits EOS is still retired within a few steps: the argmax
    marks its slot finished on the device and the count reaching the host triggers an early readback. Tokens equal
    the eager decode cut at EOS (graph mode drops the EOS token)."""
    # N(0, 1) weights: greedy streams that keep finding new tokens, with top-2 logit margins >= 0.09 (checked
    # with the oracle), so every request gets an EOS position several steps in.
    m = random_model(cuda, 405, vocab_size=100).init_normal_(1.0, seed=405)
    gen = torch.Generator().manual_seed(405)
    mels = [torch.randn(80, 150 + 20 * i, generator=gen).to(cuda) for i in range(6)]
    prompt = torch.tensor([[1, 2]])

    def run(graph, eos_ids, k=16):
        enc, dec = pools(m, cuda)
        kw = dict(graph_decode=True, graph_readback_k=k) if graph else {}
        s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=8, device=str(cuda), **kw)
        for mel, e in zip(mels, eos_ids):
            s.submit(mel, prompt_token_ids=prompt, max_new_tokens=40, eos_token_id=e)
        done = sorted(s.run_until_done(), key=lambda r: r.id)
        assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0
        return done, s

    base, _ = run(False, [-1] * 6)
    # Per request, the EOS id is the token at the last position >= 2 where a token first appears, so the
    # request stops there (graph mode keeps the tokens before it).
    eos_ids, cut = [], []
    for r in base:
        toks = r.generated_tokens
        firsts = [p for p in range(2, len(toks)) if toks[p] not in toks[:p]]
        pos = firsts[-1] if firsts else None
        eos_ids.append(toks[pos] if pos is not None else -1)
        cut.append(toks[:pos] if pos is not None else toks)
    assert sum(e >= 0 for e in eos_ids) >= 5, ("seeded model gives too few usable EOS positions",
                                               [r.generated_tokens for r in base])
    done, s = run(True, eos_ids)
    assert [r.generated_tokens for r in done] == cut
    extra = [r.graph_extra_slot_steps for r, e in zip(done, eos_ids) if e >= 0]
    assert max(extra) <= 5, extra          # the 16-step window alone would allow up to 15
    assert s.graph_buffers.early_readbacks > 0


def test_graph_slots_reused_across_lengths(cuda):
    m = random_model(cuda, 202, vocab_size=100)
    enc, dec = pools(m, cuda)
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda),
                                  graph_decode=True, graph_readback_k=4)
    gen = torch.Generator().manual_seed(202)
    lengths = [5, 15, 8, 20, 6, 12]
    for i, n in enumerate(lengths):
        s.submit(torch.randn(80, 100 + 30 * i, generator=gen).to(cuda), prompt_token_ids=torch.tensor([[1, 2]]),
                 max_new_tokens=n)
    done = s.run_until_done()
    assert len(done) == 6 and all(len(r.generated_tokens) <= r.max_new_tokens for r in done)
    assert any(r.graph_slot_reused for r in done)
    assert dec.num_free_blocks == 128 and enc.num_free_blocks == 128 and s.graph_buffers.active_slot_count() == 0


def test_failed_decode_step_releases_everything(cuda):
    m = random_model(cuda, 7)
    enc, dec = pools(m, cuda)
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda))
    real = m.decode_step_paged
    calls = [0]

    def flaky(*a, **k):
        calls[0] += 1
        if calls[0] == 4:  # one batched prefill of both requests, 2 decode steps, then fail
            raise RuntimeError("injected failure")
        return real(*a, **k)

    m.decode_step_paged = flaky
    for i in range(2):
        s.submit(torch.randn(80, 64).to(cuda), max_new_tokens=10)
    done = s.run_until_done()
    assert len(done) == 2 and all(r.phase == RequestPhase.FAILED for r in done)
    assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0
    assert s.cross_arena.owner == [] and s.cross_arena.lens == []


@pytest.mark.parametrize("mode", ["eager", "graph"])
def test_failed_batched_prefill_fails_its_requests_and_releases_everything(cuda, mode):
    """A prefill batch that raises fails the requests of that batch (blocks, arena and graph slots all
    returned); a request admitted afterwards decodes normally."""
    m = random_model(cuda, 8)
    enc, dec = pools(m, cuda)
    kw = dict(graph_decode=True, graph_readback_k=4, graph_direct_encoder_kv=True) if mode == "graph" else {}
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda), **kw)
    real = m.decode_step_paged
    calls = [0]

    def flaky(*a, **k):
        calls[0] += 1
        if calls[0] == 1:
            raise RuntimeError("injected prefill failure")
        return real(*a, **k)

    m.decode_step_paged = flaky
    for _ in range(3):
        s.submit(torch.randn(80, 64).to(cuda), max_new_tokens=6)
    s.step()
    assert len(s.completed) == 3 and all(r.phase == RequestPhase.FAILED for r in s.completed)
    assert not s.active_encode and not s.active_decode
    assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0
    if mode == "graph":
        assert s.graph_buffers.active_slot_count() == 0
    else:
        assert s.cross_arena.owner == [] and s.cross_arena.lens == []
    s.submit(torch.randn(80, 64).to(cuda), max_new_tokens=6)
    done = s.run_until_done()
    assert done[-1].phase == RequestPhase.COMPLETED and len(done[-1].generated_tokens) == 6
    assert dec.allocated_block_count == 0 and enc.allocated_block_count == 0


def test_config1_tiny_greedy_tokens_match_oracle(cuda):
    """Whisper-tiny-shaped decoder, fp32 N(0, 0.02) weights: 4 layers, d_model 384,
    4 heads x 64, vocab 51865, batch 4, 1500 N(0,1) encoder positions projected by
    cross_attn_k/v, block size 16, greedy 64 tokens from the 4-token Whisper prompt."""
    m = WhisperClassSpeechEncoderDecoderModel(4, 4, 4, 384, 80, 51865, head_dim=64).init_normal_(0.02, seed=1)
    m = m.to(cuda).eval()
    om = oracle_of(m)
    gen = torch.Generator().manual_seed(11)
    states = [torch.randn(1, 1500, 384, generator=gen) for _ in range(4)]
    prompt = [50258, 50259, 50359, 50363]
    want = [om.greedy(prompt, om.project_cross_kv(st.numpy().astype(np.float64)), 64)[0] for st in states]
    for graph in (False, True):
        enc, dec = pools(m, cuda, enc_blocks=16, dec_blocks=64)
        kw = dict(graph_decode=True, graph_readback_k=4, graph_direct_encoder_kv=True) if graph else {}
        s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), max_batch_size=4, device=str(cuda),
                                      eos_token_id=-1, **kw)
        with torch.no_grad():
            for st in states:
                s.submit_encoded(m.project_cross_kv(st.to(cuda)), prompt_token_ids=torch.tensor([prompt]),
                                 max_new_tokens=64)
        got = [r.generated_tokens for r in sorted(s.run_until_done(), key=lambda r: r.id)]
        assert got == want, f"graph={graph}"
        assert dec.allocated_block_count == 0
