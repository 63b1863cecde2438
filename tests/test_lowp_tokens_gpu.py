"""fp16 / bf16 greedy decoding on the GPU against the reference's own reduced-precision decodes
(tests/golden/whisper_lowp_golden.npz: the reference's models.py cast to float16 / bfloat16 and decoded
greedily on the CPU), for the golden tiny shape, a Whisper-tiny-like decoder (4 layers, d_model 384,
4 heads x 64) and the base- and small-shaped decoders of the serving scenarios (6 layers, 512, 8 x 64;
12 layers, 768, 12 x 64), all with vocab 51865, 1500 encoder positions and the Whisper prompt. The GPU
model takes the same seeded weights and encoder K/V.

- Teacher-forced along the reference's tokens (both requests as one batch through decode_step with a
  PagedKVCache, the scheduler's eager path): at every step the top-1 logit and the top-2 margin lie within
  5 sigma of the reference's, and the GPU's argmax is the reference's token unless the reference's own
  margin is within 5 sigma (a near-tie). sigma is the rounding-error model of oracle/rounding.py summed
  over the reference's rounding sites and the paged path's (derived, not fitted). The same against float64
  math along the same path, with the paged path's sites alone.
- Free-running through the scheduler (eager and graph decode, both requests batched): the GPU's tokens are
  the reference's up to the first near-tie of the reference's decode (the whole stream when it has none).
"""
import functools

import numpy as np
import pytest
import torch

import lowp_common as LC
from oracle.rounding import Decoder64
from speech_serving.block_manager import BlockManager
from speech_serving.dual_cache_manager import DualCacheManager
from speech_serving.encoder_block_manager import EncoderBlockManager
from speech_serving.memory_guard import MemoryGuard
from speech_serving.models import PagedKVCache, WhisperClassSpeechEncoderDecoderModel
from speech_serving.phase_aware_scheduler import PhaseAwareSpeechScheduler

pytestmark = pytest.mark.gpu
Z, CFG = LC.load()
CASES = LC.cases(CFG)
BS = 16


def gpu_model(c, state, cuda, dtype):
    m = WhisperClassSpeechEncoderDecoderModel(0, c["layers"], c["heads"], c["hidden"], 80, c["vocab"],
                                              head_dim=c["head_dim"])
    m.load_state_dict({k: v.float() for k, v in state.items()})
    return m.to(cuda, dtype).eval()


@functools.lru_cache(maxsize=None)
def setup(shape, dname):
    """The case's config, dtype, seeded weights and encoder K/V (checked against the fixture), float64
    decoder, and per request the reference's error model against the reference (both site sets) and
    against float64 (the paged sites): built once per case, shared by the tests below."""
    c = CFG["shapes"][shape]
    dt = LC.DTYPES[dname]
    names = {k: tuple(v.shape) for k, v in WhisperClassSpeechEncoderDecoderModel(
        0, c["layers"], c["heads"], c["hidden"], 80, c["vocab"], head_dim=c["head_dim"]).state_dict().items()}
    state = LC.model_state(c, names, dt)
    crosses = [LC.cross_kv(c, r, dt) for r in range(len(c["kv_seeds"]))]
    LC.check_inputs(Z, shape, dname, state, crosses)
    dec64 = Decoder64(state, c["heads"], c["head_dim"])
    keys = [f"{shape}.{dname}.r{r}" for r in range(len(crosses))]
    refs = [LC.Reference(Z, c, k, dec64, crosses[r], dt, ("reference", "paged")) for r, k in enumerate(keys)]
    exact = [LC.Reference(Z, c, k, dec64, crosses[r], dt, ("paged",), float64=True) for r, k in enumerate(keys)]
    return c, dt, state, crosses, keys, refs, exact


def teacher_forced(m, c, dt, crosses, paths, cuda):
    """GPU logits [R, steps, V] along the given token paths: the prompt's prefill, then one token per step,
    all requests as one batch through decode_step with a PagedKVCache."""
    r_n, steps, p = len(paths), len(paths[0]), len(c["prompt"])
    dec = BlockManager(c["layers"], c["heads"], c["head_dim"], BS, num_blocks=r_n * (-(-(p + steps) // BS)) + 4,
                       dtype=dt, device=str(cuda))
    tables = [[dec.allocate_block() for _ in range(-(-(p + steps) // BS))] for _ in range(r_n)]
    tab = torch.tensor(tables, dtype=torch.int32, device=cuda)
    enc = [(torch.cat([cr[l][0] for cr in crosses]).to(cuda), torch.cat([cr[l][1] for cr in crosses]).to(cuda))
           for l in range(c["layers"])]
    out = []
    with torch.no_grad():
        ids = torch.tensor([c["prompt"]] * r_n, device=cuda)
        for s in range(steps):
            n = p + s
            cache = PagedKVCache(dec.key_pool, dec.value_pool, tab,
                                 torch.full((r_n,), n, dtype=torch.int32, device=cuda), n)
            res = m.decode_step(ids, past_key_values=cache, encoder_past_kv_list=enc, use_cache=True,
                                logits_to_keep=1)
            out.append(res.logits[:, -1].double().cpu().numpy())
            ids = torch.tensor([[path[s]] for path in paths], device=cuda)
    return np.stack(out, axis=1)


@pytest.mark.parametrize("shape,dname", CASES)
def test_teacher_forced_logits_and_tokens_against_the_reference(cuda, shape, dname):
    c, dt, state, crosses, keys, refs, exact = setup(shape, dname)
    m = gpu_model(c, state, cuda, dt)
    got = teacher_forced(m, c, dt, crosses, [ref.tokens for ref in refs], cuda)
    for r, (ref, ex) in enumerate(zip(refs, exact)):
        a = LC.compare(ref, got[r], f"GPU vs the reference's {keys[r]}")
        b = LC.compare(ex, got[r], f"GPU vs float64 along {keys[r]}")
        print(f"{keys[r]}: GPU argmax = the reference's token at {a['argmax_equal']}/{a['steps']} steps "
              f"(near-ties {a['near_ties']}); = float64 argmax at {b['argmax_equal']}/{b['steps']} "
              f"(near-ties {b['near_ties']}); median sigma {np.median(ref.sigma_top):.2e} / {np.median(ex.sigma_top):.2e}")


@pytest.mark.parametrize("mode", ["eager", "graph"])
@pytest.mark.parametrize("shape,dname", CASES)
def test_free_running_tokens_follow_the_reference(cuda, shape, dname, mode):
    c, dt, state, crosses, keys, refs, _ = setup(shape, dname)
    m = gpu_model(c, state, cuda, dt)
    steps = len(Z[f"{shape}.{dname}.r0.tokens"])
    pool = len(crosses) * (-(-(len(c["prompt"]) + steps) // BS)) + 8
    dec = BlockManager(c["layers"], c["heads"], c["head_dim"], BS, num_blocks=pool, dtype=dt, device=str(cuda))
    enc = EncoderBlockManager(1, c["heads"], c["head_dim"], BS, num_blocks=8, dtype=dt, device=str(cuda))
    kw = dict(graph_decode=True, graph_readback_k=4, graph_direct_encoder_kv=True,
              graph_max_enc_len=c["t_enc"]) if mode == "graph" else {}
    s = PhaseAwareSpeechScheduler(m, DualCacheManager(enc, dec), MemoryGuard(high_water_mark_pct=1e9),
                                  max_batch_size=len(crosses), device=str(cuda), eos_token_id=-1, **kw)
    for cross in crosses:
        s.submit_encoded([(k.to(cuda), v.to(cuda)) for k, v in cross], prompt_token_ids=torch.tensor([c["prompt"]]),
                         max_new_tokens=steps)
    done = sorted(s.run_until_done(), key=lambda q: q.id)
    assert dec.allocated_block_count == 0
    for r, q in enumerate(done):
        key, ref = keys[r], refs[r]
        ties = np.nonzero(ref.near_tie)[0]
        limit = int(ties[0]) if ties.size else steps  # the steps before the reference's first near-tie
        same = 0
        while same < steps and q.generated_tokens[same] == ref.tokens[same]:
            same += 1
        assert len(q.generated_tokens) == steps
        assert same >= limit, f"{key} {mode}: tokens differ at step {same}, before the first near-tie ({limit})"
        print(f"{key} {mode}: {same}/{steps} tokens identical to the reference's decode "
              f"(first near-tie at step {int(ties[0]) if ties.size else None})")
