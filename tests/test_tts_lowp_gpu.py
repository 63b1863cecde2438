"""fp16 / bf16 streaming TTS on the GPU against the reference's own reduced-precision decodes
(tests/golden/tts_lowp_golden.npz: the reference's StreamingMultiCodebookTTSModel cast to float16 /
bfloat16 and decoded greedily on the CPU), for the float32 golden shape (2 layers, 4 heads x 16, 4
codebooks, vocab 128) and the reference model's default shape (4 layers, 4 heads x 64, 4 codebooks,
vocab 1024). The GPU model takes the same seeded weights and prompts.

- Teacher-forced along the reference's frames (both requests as one batch through the model's forward
  with a PagedKVCache, the engine's step): for every (frame, codebook) the top-1 logit and the top-2
  margin lie within 5 sigma of the reference's, and the GPU's code is the reference's unless the
  reference's own margin is within 5 sigma (a near-tie); sigma from the rounding model of
  oracle/rounding.py over the reference's and the paged path's rounding sites (derived, not fitted).
  The same against float64 math along the same path, with the paged path's sites alone.
- Free-running through the engine (eager and graph decode, both requests batched): the frames are the
  reference's up to the first frame with a near-tie in any codebook (every frame when there is none).
"""
import functools

import numpy as np
import pytest
import torch

import tts_lowp_common as TC
from oracle.rounding import MultiCodebook64
from speech_serving.block_manager import BlockManager
from speech_serving.models import PagedKVCache, StreamingMultiCodebookTTSModel
from speech_serving.tts_engine import StreamingTTSEngine

pytestmark = pytest.mark.gpu
Z, CFG = TC.load()
CASES = TC.cases(CFG)
BS = 16


@functools.lru_cache(maxsize=None)
def setup(shape, dname):
    """The case's config, dtype, seeded weights (checked against the fixture) and per request the error
    models against the reference (both site sets) and against float64 (the paged sites): once per case."""
    c = CFG["shapes"][shape]
    dt = TC.DTYPES[dname]
    names = {k: tuple(v.shape) for k, v in StreamingMultiCodebookTTSModel(**TC.model_args(c)).state_dict().items()}
    state = TC.model_state(c, names, dt)
    TC.check_state(Z, shape, dname, state)
    mc = MultiCodebook64(state, c["num_heads"], c["hidden_dim"] // c["num_heads"])
    keys = [f"{shape}.{dname}.r{r}" for r in range(len(c["prompt_seeds"]))]
    refs = [TC.TTSReference(Z, c, k, mc, dt, ("reference", "paged")) for k in keys]
    exact = [TC.TTSReference(Z, c, k, mc, dt, ("paged",), float64=True) for k in keys]
    return c, dt, state, keys, refs, exact


def gpu_model(c, state, cuda, dtype):
    m = StreamingMultiCodebookTTSModel(**TC.model_args(c))
    m.load_state_dict({k: v.float() for k, v in state.items()})
    return m.to(cuda, dtype).eval()


def block_manager(c, dt, cuda, blocks):
    return BlockManager(c["num_layers"], c["num_heads"], c["hidden_dim"] // c["num_heads"], BS, num_blocks=blocks,
                        dtype=dt, device=str(cuda))


def teacher_forced(m, c, dt, refs, cuda):
    """GPU logits per request [F * K, V] along the reference's frames: the prompts' prefill, then one frame
    per step, both requests as one batch through forward with a PagedKVCache."""
    r_n, f_n, p = len(refs), len(refs[0].frames), len(refs[0].prompt)
    nblk = -(-(p + f_n) // BS)
    bm = block_manager(c, dt, cuda, r_n * nblk + 4)
    tab = torch.tensor([[bm.allocate_block() for _ in range(nblk)] for _ in range(r_n)], dtype=torch.int32,
                       device=cuda)
    out = []
    with torch.no_grad():
        codes = torch.tensor([ref.prompt for ref in refs], device=cuda)
        for s in range(f_n):
            n = p + s
            cache = PagedKVCache(bm.key_pool, bm.value_pool, tab, torch.full((r_n,), n, dtype=torch.int32,
                                                                             device=cuda), n)
            res = m(codes, past_key_values=cache, logits_to_keep=1)
            out.append(res.logits[:, -1].double().cpu().numpy())  # [R, K, V]
            codes = torch.tensor([[ref.frames[s]] for ref in refs], device=cuda)
    got = np.stack(out, axis=1)  # [R, F, K, V]
    return [g.reshape(f_n * c["num_codebooks"], c["vocab_size"]) for g in got]


@pytest.mark.parametrize("shape,dname", CASES)
def test_teacher_forced_logits_and_codes_against_the_reference(cuda, shape, dname):
    c, dt, state, keys, refs, exact = setup(shape, dname)
    got = teacher_forced(gpu_model(c, state, cuda, dt), c, dt, refs, cuda)
    for r, (ref, ex) in enumerate(zip(refs, exact)):
        a = TC.compare(ref, got[r], f"GPU vs the reference's {keys[r]}")
        b = TC.compare(ex, got[r], f"GPU vs float64 along {keys[r]}")
        print(f"{keys[r]}: GPU code = the reference's at {a['argmax_equal']}/{a['steps']} (frame, codebook) rows "
              f"(near-ties {a['near_ties']}); = float64 argmax at {b['argmax_equal']}/{b['steps']} "
              f"(near-ties {b['near_ties']}); median sigma {np.median(ref.sigma_top):.2e} / {np.median(ex.sigma_top):.2e}")


@pytest.mark.parametrize("mode", ["eager", "graph"])
@pytest.mark.parametrize("shape,dname", CASES)
def test_free_running_frames_follow_the_reference(cuda, shape, dname, mode):
    c, dt, state, keys, refs, _ = setup(shape, dname)
    m = gpu_model(c, state, cuda, dt)
    f_n, p = len(refs[0].frames), len(refs[0].prompt)
    bm = block_manager(c, dt, cuda, len(refs) * -(-(p + f_n) // BS) + 8)
    engine = StreamingTTSEngine(m, bm, max_batch_size=len(refs), device=str(cuda), graph_decode=mode == "graph")
    for ref in refs:
        engine.submit(torch.tensor(ref.prompt), max_new_frames=f_n)
    done = sorted(engine.run_until_done(), key=lambda q: q.id)
    assert bm.allocated_block_count == 0
    k_n = c["num_codebooks"]
    for r, q in enumerate(done):
        ref = refs[r]
        frames = [f.tolist() for f in q.generated_frames]
        assert len(frames) == f_n
        tie_frames = sorted({int(i) // k_n for i in np.nonzero(ref.near_tie)[0]})
        limit = tie_frames[0] if tie_frames else f_n  # the frames before the reference's first near-tie
        same = 0
        while same < f_n and frames[same] == ref.frames[same]:
            same += 1
        assert same >= limit, f"{keys[r]} {mode}: frames differ at {same}, before the first near-tie ({limit})"
        print(f"{keys[r]} {mode}: {same}/{f_n} frames identical to the reference's decode "
              f"(first near-tie at frame {tie_frames[0] if tie_frames else None})")
