"""The reduced-precision error model (oracle/rounding.py) against the reference's own fp16 / bf16 decodes
(tests/golden/whisper_lowp_golden.npz, written from the reference's models.py on the CPU):

- the float64 restatement Decoder64 equals the float64 oracle (oracle/decoder.py, pinned by the
  reference's float32 golden vectors) on the golden model, teacher-forced;
- the seeded weights and encoder K/V regenerate bit for bit (the fixture's checksums);
- the reference's fp16 / bf16 logits lie within 5 sigma of float64 math along the reference's token path,
  sigma from the reference's own rounding sites (every op output), and the float64 argmax equals the
  reference's token except at near-ties;
- the rounding emulation that rounds where the reference rounds reproduces the reference's logits
  (bit for bit on every tiny-shape fixture: the top-16 logits of every step, and all 100 logits of every step
  of at least two of them), while a misplaced set of rounding sites (the paged path's, which keeps attention
  scores and probabilities in fp32) does not: the site list is pinned by the reference's arithmetic. At the
  larger shapes (Whisper-tiny-like, base- and small-shaped) the reference's fp32 accumulation order moves
  logits by a few dtype steps whichever sites are rounded, so there the emulation is held to the reference's
  rounding model (its logits within 5 sigma, its tokens the reference's except at near-ties).
"""
import json
import os

import numpy as np
import pytest
import torch

import lowp_common as LC
from oracle import decoder as D
from oracle.rounding import Decoder64, round_through, ulp
from speech_serving.models import WhisperClassSpeechEncoderDecoderModel

GOLDEN32 = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "whisper_tiny_golden.npz")


def shapes_of(c):
    m = WhisperClassSpeechEncoderDecoderModel(0, c["layers"], c["heads"], c["hidden"], 80, c["vocab"],
                                              head_dim=c["head_dim"])
    return {k: tuple(v.shape) for k, v in m.state_dict().items()}


def test_decoder64_equals_the_float64_oracle():
    z = np.load(GOLDEN32, allow_pickle=False)
    cfg = json.loads(bytes(z["config_json"]).decode())
    state = {k[len("param."):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param.")}
    om = D.Model({k: v.numpy() for k, v in state.items()}, cfg["num_heads"], cfg["hidden_dim"] // cfg["num_heads"])
    cross = [(z[f"enc_k{l}"], z[f"enc_v{l}"]) for l in range(cfg["num_encoder_layers"])]
    ids = cfg["prompt"] + z["greedy_tokens"].tolist()
    want, _ = om.decode_step(np.asarray([ids]), None, cross)
    dec = Decoder64(state, cfg["num_heads"], cfg["hidden_dim"] // cfg["num_heads"])
    got = dec.forward(ids, [(torch.from_numpy(k), torch.from_numpy(v)) for k, v in cross])
    np.testing.assert_allclose(got.numpy(), want[0], rtol=0, atol=1e-10)
    # and the recorded sites are the values the forward used
    sites = {}
    again = dec.forward(ids, [(torch.from_numpy(k), torch.from_numpy(v)) for k, v in cross], sites)
    assert torch.equal(again.detach(), got) and torch.equal(sites["logits"].detach(), got)
    assert {n.split(".", 1)[1] for n in sites if "." in n} == {
        "norm1", "q", "k", "v", "scores", "probs", "attn", "attn_out", "res1", "norm2", "cq", "cscores", "cprobs",
        "cattn", "cattn_out", "res2", "norm3", "fc1", "gelu", "fc2", "res3"}


@pytest.fixture(scope="module")
def lowp():
    z, cfg = LC.load()
    out = {}
    for shape, dname in LC.cases(cfg):
        c = cfg["shapes"][shape]
        dt = LC.DTYPES[dname]
        state = LC.model_state(c, shapes_of(c), dt)
        crosses = [LC.cross_kv(c, r, dt) for r in range(len(c["kv_seeds"]))]
        LC.check_inputs(z, shape, dname, state, crosses)
        dec = Decoder64(state, c["heads"], c["head_dim"])
        refs = [LC.Reference(z, c, f"{shape}.{dname}.r{r}", dec, crosses[r], dt, ("reference",))
                for r in range(len(crosses))]
        out[(shape, dname)] = (c, dt, dec, crosses, refs)
    return z, cfg, out


def test_reference_lowp_decodes_within_the_rounding_model(lowp):
    z, cfg, cases = lowp
    for (shape, dname), (c, dt, dec, crosses, refs) in cases.items():
        for r, ref in enumerate(refs):
            stats = LC.compare(ref, ref.logits64, f"float64 vs reference {shape}.{dname}.r{r}")
            print(f"{shape} {dname} r{r}: float64 argmax = reference token at {stats['argmax_equal']}/{stats['steps']} "
                  f"steps, near-ties {stats['near_ties']}, median sigma(top logit) {np.median(ref.sigma_top):.2e}")


def test_rounding_emulation_reproduces_the_reference(lowp):
    z, cfg, cases = lowp
    exact_cases = full_exact = 0
    for (shape, dname), (c, dt, dec, crosses, refs) in cases.items():
        for r, ref in enumerate(refs):
            key = f"{shape}.{dname}.r{r}"
            em = {pl: round_through(dec, ref.ids, crosses[r], dt, pl)[ref.positions] for pl in ("reference", "paged")}
            got = {pl: np.take_along_axis(e.numpy(), ref.top_idx, axis=1) for pl, e in em.items()}
            steps = {pl: np.abs(g - ref.top_val) / ulp(torch.from_numpy(ref.top_val), dt).numpy()
                     for pl, g in got.items()}
            # The emulation differs from the reference only by the reference's fp32 accumulation order: its
            # logits lie within the reference's own rounding model, and its tokens are the reference's except
            # at near-ties.
            LC.compare(ref, em["reference"].numpy(), f"reference-site emulation vs {key}")
            print(f"{key}: logits equal to the reference's bit for bit: {(steps['reference'] == 0).mean():.3f} "
                  f"(misplaced sites {(steps['paged'] == 0).mean():.3f}); largest gap {steps['reference'].max():.0f} "
                  f"dtype steps (misplaced sites {steps['paged'].max():.0f})")
            if shape == "tiny":
                # sums short enough that the reference's fp32 accumulation order does not show: the site list
                # decides, and only the reference's sites reproduce its logits
                assert (steps["reference"] == 0).mean() > (steps["paged"] == 0).mean(), key
                if (steps["reference"] == 0).all():
                    exact_cases += 1
                    assert (steps["paged"] > 0).any(), key
                    full = z[f"{key}.logits"].astype(np.float64)
                    full_exact += int(np.array_equal(em["reference"].numpy(), full))
    # every tiny-shape fixture: the top-16 logits of every step bit for bit (all 100 logits of every step in at
    # least two of them)
    assert exact_cases == 4 and full_exact >= 2
