"""StreamingTTSEngine / StreamingMultiCodebookTTSModel on the paged kernels.

- The reference's own TTS test (test_speech_engine.py:35-91), unchanged in substance.
- Parity with the reference: the golden file tests/golden/tts_small_golden.npz (written from
  the reference model and engine, CPU float32) holds the weights, prompts, prefill logits and
  K/V, the logits of every generated frame and the engine's frames. Here the same weights run
  in float32 on the GPU: frames must be identical, logits within 1e-4 (the golden seed keeps
  every greedy margin above 2.7e-3), the prefill K/V written into the pool within 1e-5.
- Bookkeeping: every request's block table after each frame equals the oracle engine's
  (oracle/tts.py, LIFO free list), all blocks return to the pool.
- Failure paths: a raising frame callback only warns; running out of blocks mid-decode ends
  that request alone.
- Graph decode (the default) gives the eager engine's frames, also with staggered requests that
  reuse slots, change batch buckets and outgrow the captured context cap, and its captured graphs
  survive a later growth of the attention workspace.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle.tts import Engine
from speech_serving import BlockManager, StreamingMultiCodebookTTSModel, StreamingTTSEngine
from speech_serving.models import PagedKV

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "tts_small_golden.npz")


def _golden(device):
    z = np.load(GOLDEN)
    cfg = json.loads(bytes(z["config_json"]).decode())
    model = StreamingMultiCodebookTTSModel(cfg["num_layers"], cfg["num_heads"], cfg["hidden_dim"],
                                           cfg["num_codebooks"], cfg["vocab_size"])
    state = {k[len("param."):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param.")}
    model.load_state_dict(state, strict=True)
    return z, cfg, model.to(device=device, dtype=torch.float32).eval()


def _bm(cfg, device, dtype=torch.float32, num_blocks=None):
    return BlockManager(num_layers=cfg["num_layers"], num_kv_heads=cfg["num_heads"],
                        head_dim=cfg["hidden_dim"] // cfg["num_heads"], block_size=cfg["block_size"],
                        num_blocks=num_blocks or cfg["num_blocks"], dtype=dtype, device=str(device))


def test_reference_streaming_tts_engine(cuda):
    """test_speech_engine.py:35-91: 3 requests x 15 frames, batch 2, block size 8, 32 blocks, fp16."""
    num_layers, num_heads, hidden_dim, num_codebooks, vocab_size, block_size = 2, 4, 64, 4, 128, 8
    torch.manual_seed(0)
    model = StreamingMultiCodebookTTSModel(num_layers=num_layers, num_heads=num_heads, hidden_dim=hidden_dim,
                                           num_codebooks=num_codebooks, vocab_size=vocab_size)
    model = model.to(device=cuda, dtype=torch.float16).eval()
    bm = BlockManager(num_layers=num_layers, num_kv_heads=num_heads, head_dim=hidden_dim // num_heads,
                      block_size=block_size, num_blocks=32, dtype=torch.float16, device=str(cuda))
    engine = StreamingTTSEngine(model, bm, max_batch_size=2, device=str(cuda))
    frames_received = {}

    def callback_factory(req_id):
        def cb(rid, frame):
            assert rid == req_id and frame.shape == (num_codebooks,) and frame.dtype == torch.int64
            frames_received[rid] = frames_received.get(rid, 0) + 1
        return cb

    for i in range(3):
        prompt = torch.randint(0, vocab_size, (10, num_codebooks), device=cuda)
        engine.submit(prompt, max_new_frames=15, on_frame_callback=callback_factory(i))
    completed = engine.run_until_done()

    assert len(completed) == 3
    for req in completed:
        assert req.done
        assert req.generated_count == 15
        assert len(req.generated_frames) == 15
        assert req.generated_frames[0].shape[0] == num_codebooks
        assert all(int(f.min()) >= 0 and int(f.max()) < vocab_size for f in req.generated_frames)
    assert frames_received == {0: 15, 1: 15, 2: 15}
    assert bm.allocated_block_count == 0
    assert bm.num_free_blocks == 32


@pytest.mark.parametrize("graph", [False, True])
def test_frames_match_reference_engine(cuda, graph):
    z, cfg, model = _golden(cuda)
    bm = _bm(cfg, cuda)
    engine = StreamingTTSEngine(model, bm, max_batch_size=cfg["max_batch"], device=str(cuda), graph_decode=graph)
    tables = {}
    emit = engine._emit

    def record(req, frame):
        tables.setdefault(req.id, []).append(list(req.block_table))
        return emit(req, frame)

    engine._emit = record
    for r in range(cfg["requests"]):
        engine.submit(torch.from_numpy(z["prompts"][r]), max_new_frames=cfg["frames"])
    done = engine.run_until_done()
    assert [q.id for q in done] == [0, 1, 2]
    for q in done:
        got = torch.stack(q.generated_frames).cpu().numpy()
        assert np.array_equal(got, z[f"engine_frames{q.id}"]), q.id
    assert [bm.allocated_block_count, bm.num_free_blocks] == z["engine_blocks"].tolist()
    _, history, _ = Engine(cfg["num_blocks"], cfg["block_size"], cfg["max_batch"]).run(
        [cfg["prompt_len"]] * cfg["requests"], [cfg["frames"]] * cfg["requests"])
    assert tables == history


class HookOnlyTTSModel:
    """A TTS model that offers the engine only the reference's call, model(input_codebooks,
    past_key_values, use_cache) on contiguous K/V (tts_engine.py:188), and the attributes it reads."""

    def __init__(self, m):
        self._m = m
        for a in ("num_layers", "num_heads", "head_dim", "hidden_dim", "num_codebooks", "vocab_size", "config"):
            setattr(self, a, getattr(m, a))
        self.calls = 0

    def __call__(self, input_codebooks, past_key_values=None, use_cache=True):
        self.calls += 1
        return self._m(input_codebooks, past_key_values=past_key_values, use_cache=use_cache)


def test_hook_only_model_frames_match_reference_engine(cuda):
    """A model with only the reference's forward is served as the reference serves it (per request:
    history gathered out of the pool, forward, new K/V appended): the golden frames and block tables;
    graph decode, which captures the paged step, refuses it."""
    z, cfg, m = _golden(cuda)
    bm = _bm(cfg, cuda)
    model = HookOnlyTTSModel(m)
    with pytest.raises(TypeError, match="graph_decode=False"):
        StreamingTTSEngine(model, bm, max_batch_size=cfg["max_batch"], device=str(cuda), graph_decode=True)
    engine = StreamingTTSEngine(model, bm, max_batch_size=cfg["max_batch"], device=str(cuda))
    assert not engine.graph_decode
    for r in range(cfg["requests"]):
        engine.submit(torch.from_numpy(z["prompts"][r]), max_new_frames=cfg["frames"])
    done = engine.run_until_done()
    assert [q.id for q in done] == [0, 1, 2]
    for q in done:
        assert np.array_equal(torch.stack(q.generated_frames).cpu().numpy(), z[f"engine_frames{q.id}"]), q.id
    assert model.calls == cfg["requests"] * cfg["frames"]  # one prefill and frames - 1 steps per request
    assert [bm.allocated_block_count, bm.num_free_blocks] == z["engine_blocks"].tolist()


def test_forward_wrapper_sees_every_eager_step(cuda):
    """Eager decode of a paged model goes through model(...) too: a wrapper that forces codebook 0 to
    token 3 from the second call on changes every later frame's first token, as it would in the
    reference's engine."""
    z, cfg, m = _golden(cuda)
    bm = _bm(cfg, cuda)
    engine = StreamingTTSEngine(m, bm, max_batch_size=cfg["max_batch"], device=str(cuda), graph_decode=False)
    real = m.forward
    n = [0]

    def forced(*a, **k):
        out = real(*a, **k)
        n[0] += 1
        if n[0] >= 2:
            out.logits[:, -1, 0, :] = -1e4
            out.logits[:, -1, 0, 3] = 1e4
        return out

    m.forward = forced
    engine.submit(torch.from_numpy(z["prompts"][0]), max_new_frames=cfg["frames"])
    (q,) = engine.run_until_done()
    m.forward = real
    frames = torch.stack(q.generated_frames).cpu().numpy()
    assert n[0] == cfg["frames"]
    assert (frames[1:, 0] == 3).all()
    assert np.array_equal(frames[0], z["engine_frames0"][0])


def test_prefill_and_step_logits_match_reference(cuda):
    z, cfg, model = _golden(cuda)
    bm = _bm(cfg, cuda)
    bs = cfg["block_size"]
    for r in range(cfg["requests"]):
        prompt = torch.from_numpy(z["prompts"][r]).to(cuda)
        p = prompt.shape[0]
        blocks = [bm.allocate_block() for _ in range(-(-(p + cfg["frames"]) // bs))]
        table = torch.tensor([blocks], dtype=torch.int32, device=cuda)

        def kv(n):
            return PagedKV(bm.key_pool, bm.value_pool, table, torch.tensor([n], dtype=torch.int32, device=cuda), n)

        with torch.no_grad():
            logits = model.decode_step_paged(prompt[None], kv(p), last_only=False)  # [1, P, K, V]
            np.testing.assert_allclose(logits.cpu().numpy(), z[f"prefill_logits{r}"], atol=1e-4, rtol=0)
            if r == 0:
                for l in range(cfg["num_layers"]):
                    for pool, key in ((bm.key_pool[l], "prefill_k"), (bm.value_pool[l], "prefill_v")):
                        got = pool[blocks].reshape(-1, cfg["num_heads"], pool.shape[-1])[:p].permute(1, 0, 2)
                        np.testing.assert_allclose(got.cpu().numpy(), z[f"{key}{l}"][0], atol=1e-5, rtol=0)
            want = z[f"step_logits{r}"]
            last = logits[:, -1]
            n = p
            for f in range(cfg["frames"]):
                np.testing.assert_allclose(last[0].cpu().numpy(), want[f], atol=1e-4, rtol=0, err_msg=f"r{r} f{f}")
                nxt = last.argmax(-1)[:, None, :]  # [1, 1, K]
                n += 1
                last = model.decode_step_paged(nxt, kv(n))
        bm.free_blocks(blocks)
    assert bm.allocated_block_count == 0


def test_raising_callback_only_warns(cuda, capsys):
    z, cfg, model = _golden(cuda)
    bm = _bm(cfg, cuda)
    engine = StreamingTTSEngine(model, bm, max_batch_size=2, device=str(cuda))

    def bad(rid, frame):
        raise ValueError("listener gone")

    engine.submit(torch.from_numpy(z["prompts"][0]), max_new_frames=4, on_frame_callback=bad)
    done = engine.run_until_done()
    assert len(done) == 1 and done[0].generated_count == 4
    assert np.array_equal(torch.stack(done[0].generated_frames).cpu().numpy(), z["engine_frames0"][:4])
    assert "Exception in frame callback" in capsys.readouterr().out
    assert bm.allocated_block_count == 0


@pytest.mark.parametrize("graph", [False, True])
def test_out_of_blocks_mid_decode_ends_that_request(cuda, capsys, graph):
    """4 blocks of 8: two 10-frame prompts take 2 blocks each; the first to need a third block
    (sequence length 16) fails and is released, after which the other one continues."""
    z, cfg, model = _golden(cuda)
    bm = _bm(cfg, cuda, num_blocks=4)
    engine = StreamingTTSEngine(model, bm, max_batch_size=2, device=str(cuda), graph_decode=graph)
    for r in range(2):
        engine.submit(torch.from_numpy(z["prompts"][r]), max_new_frames=cfg["frames"])
    done = engine.run_until_done()
    out = capsys.readouterr().out
    assert "Error executing step for TTS request 0" in out
    assert [q.id for q in done] == [0, 1]
    assert done[0].generated_count == 7  # frames 1..7 at sequence lengths 10..16, the 8th needs block 3
    assert done[1].generated_count == cfg["frames"]
    assert np.array_equal(torch.stack(done[1].generated_frames).cpu().numpy(), z["engine_frames1"])
    assert np.array_equal(torch.stack(done[0].generated_frames).cpu().numpy(), z["engine_frames0"][:7])
    assert bm.allocated_block_count == 0 and bm.num_free_blocks == 4


def _run(model, cfg, cuda, requests, graph, max_batch, num_blocks, before_step=None):
    bm = _bm(cfg, cuda, num_blocks=num_blocks)
    engine = StreamingTTSEngine(model, bm, max_batch_size=max_batch, device=str(cuda), graph_decode=graph)
    for prompt, frames in requests:
        engine.submit(prompt, max_new_frames=frames)
    steps = 0
    while engine.active or engine.queue:
        if before_step is not None:
            before_step(steps)
        engine.step()
        steps += 1
    out = {q.id: torch.stack(q.generated_frames).cpu().numpy() for q in engine.completed}
    assert bm.allocated_block_count == 0
    return out, engine


def _staggered(cfg, n=7, seed=5):
    g = torch.Generator().manual_seed(seed)
    reqs = []
    for i in range(n):
        p = int(torch.randint(1, 40, (1,), generator=g))
        f = int(torch.randint(1, 30, (1,), generator=g))
        reqs.append((torch.randint(0, cfg["vocab_size"], (p, cfg["num_codebooks"]), generator=g), f))
    reqs.append((torch.randint(0, cfg["vocab_size"], (240, cfg["num_codebooks"]), generator=g), 40))  # past 256
    return reqs


def test_graph_decode_matches_eager_with_slot_reuse_and_cap_growth(cuda):
    z, cfg, model = _golden(cuda)
    reqs = _staggered(cfg)
    eager, _ = _run(model, cfg, cuda, reqs, False, 4, 128)
    graph, eng = _run(model, cfg, cuda, reqs, True, 4, 128)
    assert eng._cap >= 512  # the 240-frame prompt outgrew the first cap
    assert sorted(graph) == sorted(eager) == list(range(len(reqs)))
    for r in eager:
        assert graph[r].shape == (reqs[r][1], cfg["num_codebooks"])
        assert np.array_equal(graph[r], eager[r]), r


def test_graphs_survive_workspace_growth(cuda):
    """The captured graphs keep the attention workspace they were captured with alive: after an
    eager call grows the device's workspace, replays still produce the eager frames and do not
    write into memory handed out after the growth."""
    from speech_serving import native

    z, cfg, model = _golden(cuda)
    reqs = [(torch.from_numpy(z["prompts"][r]), cfg["frames"]) for r in range(cfg["requests"])]
    junk = []

    def grow(step):
        if step == 3:  # graphs for the first buckets are captured by now
            ws = native.reserve_workspace(0, cuda)
            native.reserve_workspace(ws.numel() * 4, cuda)
            for _ in range(8):  # fresh allocations that could land on the old workspace
                junk.append(torch.full((ws.numel() // 4,), 7, dtype=torch.int32, device=cuda))

    graph, _ = _run(model, cfg, cuda, reqs, True, cfg["max_batch"], cfg["num_blocks"], before_step=grow)
    for r in range(cfg["requests"]):
        assert np.array_equal(graph[r], z[f"engine_frames{r}"]), r
    assert junk and all(bool((t == 7).all()) for t in junk)
