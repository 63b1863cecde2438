"""The reduced-precision error model over the streaming TTS model (oracle/rounding.MultiCodebook64)
against the reference's own fp16 / bf16 decodes (tests/golden/tts_lowp_golden.npz, written from the
reference's models.py on the CPU):

- the float64 restatement MultiCodebook64 equals the TTS oracle (oracle/tts.py, pinned by the reference's
  float32 golden vectors) on the golden TTS model, and records the rounding sites of the embedding's partial
  sums, every layer (no cross-attention), the final norm and the heads;
- the seeded weights regenerate bit for bit (the fixture's checksums);
- the reference's fp16 / bf16 logits of every (frame, codebook) lie within 5 sigma of float64 math along its
  frame path, sigma from the reference's own rounding sites, and the float64 argmax is the reference's code
  except at near-ties;
- rounding where the reference rounds (the embedding's partial sums left to right included) reproduces the
  reference's small-shape bf16 logits bit for bit, and matches more of every small-shape fixture's top-16
  than the paged path's sites (scores and probabilities kept in fp32) do: the site list is pinned by the
  reference's arithmetic. (fp16 keeps 3 more significand bits, enough for the reference's fp32 accumulation
  order to show: 68-79% of its small-shape top-16 equal, the rest within 3 dtype steps.)
"""
import json
import os

import numpy as np
import pytest
import torch

import tts_lowp_common as TC
from oracle import tts as OT
from oracle.rounding import MultiCodebook64, round_through, ulp
from speech_serving.models import StreamingMultiCodebookTTSModel

GOLDEN32 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tts_small_golden.npz")


def shapes_of(c):
    m = StreamingMultiCodebookTTSModel(**TC.model_args(c))
    return {k: tuple(v.shape) for k, v in m.state_dict().items()}


def test_multicodebook64_equals_the_tts_oracle():
    z = np.load(GOLDEN32, allow_pickle=False)
    cfg = json.loads(bytes(z["config_json"]).decode())
    state = {k[len("param."):]: z[k] for k in z.files if k.startswith("param.")}
    h, d = cfg["num_heads"], cfg["hidden_dim"] // cfg["num_heads"]
    om = OT.TTSModel(state, h, d)
    prompt = z["prompts"][0]
    frames = prompt.tolist() + z["engine_frames0"].tolist()
    want, _ = om.forward(np.asarray([frames]))
    mc = MultiCodebook64({k: torch.from_numpy(v) for k, v in state.items()}, h, d)
    sites = {}
    got = mc.forward(frames, None, sites).detach()
    np.testing.assert_allclose(got.numpy(), want[0].reshape(len(frames), -1), rtol=0, atol=1e-10)
    assert {n.split(".", 1)[1] for n in sites if "." in n} == {
        "norm1", "q", "k", "v", "scores", "probs", "attn", "attn_out", "res1", "norm2", "fc1", "gelu", "fc2", "res3"}
    assert {n for n in sites if "." not in n} == {"emb1", "emb2", "emb3", "final_norm", "logits"}


@pytest.fixture(scope="module")
def lowp():
    z, cfg = TC.load()
    out = {}
    for shape, dname in TC.cases(cfg):
        c = cfg["shapes"][shape]
        dt = TC.DTYPES[dname]
        state = TC.model_state(c, shapes_of(c), dt)
        TC.check_state(z, shape, dname, state)
        mc = MultiCodebook64(state, c["num_heads"], c["hidden_dim"] // c["num_heads"])
        refs = [TC.TTSReference(z, c, f"{shape}.{dname}.r{r}", mc, dt, ("reference",))
                for r in range(len(c["prompt_seeds"]))]
        out[(shape, dname)] = (c, dt, mc, refs)
    return z, cfg, out


def test_reference_lowp_frames_within_the_rounding_model(lowp):
    z, cfg, cases = lowp
    for (shape, dname), (c, dt, mc, refs) in cases.items():
        for r, ref in enumerate(refs):
            stats = TC.compare(ref, ref.logits64, f"float64 vs reference {shape}.{dname}.r{r}")
            print(f"{shape} {dname} r{r}: float64 argmax = reference code at {stats['argmax_equal']}/{stats['steps']} "
                  f"(frame, codebook) rows, near-ties {stats['near_ties']}, median sigma {np.median(ref.sigma_top):.2e}")


def test_rounding_emulation_reproduces_the_reference(lowp):
    z, cfg, cases = lowp
    exact = 0
    for (shape, dname), (c, dt, mc, refs) in cases.items():
        for r, ref in enumerate(refs):
            key = f"{shape}.{dname}.r{r}"
            f_n, k_n, v_n = len(ref.frames), c["num_codebooks"], c["vocab_size"]
            pos = [len(ref.prompt) - 1 + t for t in range(f_n)]
            em = {pl: round_through(mc, ref.seq, None, dt, pl)[pos].numpy().reshape(f_n * k_n, v_n)
                  for pl in ("reference", "paged")}
            TC.compare(ref, em["reference"], f"reference-site emulation vs {key}")
            got = {pl: np.take_along_axis(e, ref.top_idx, axis=1) for pl, e in em.items()}
            steps = {pl: np.abs(g - ref.top_val) / ulp(torch.from_numpy(ref.top_val), dt).numpy()
                     for pl, g in got.items()}
            print(f"{key}: logits equal to the reference's bit for bit: {(steps['reference'] == 0).mean():.3f} "
                  f"(misplaced sites {(steps['paged'] == 0).mean():.3f}); largest gap "
                  f"{steps['reference'].max():.0f} dtype steps")
            if shape == "small":
                assert (steps["reference"] == 0).mean() > (steps["paged"] == 0).mean(), key
                full = z[f"{key}.logits"].astype(np.float64).reshape(f_n * k_n, v_n)
                exact += int(np.array_equal(em["reference"], full))
    assert exact >= 2, f"the reference-site emulation reproduced {exact} small-shape fixtures bit for bit"
