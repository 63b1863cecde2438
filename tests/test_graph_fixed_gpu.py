"""decode_step_graph_fixed — the reference's bucketed static-KV graph step (models.py:425-487, driven by
graph_decode_buffers.py:433-463 with the -10000 additive masks of :520-537) — against the reference's
golden vectors.

The golden request (3-token prompt, 8 greedy tokens, float32) runs in slot 1 of 3 static slots; the
other slots are idle (masked everywhere, as the reference's prepare_replay leaves them). The prompt is
fed one token per step, which is the causal prefill. Bars: the slot's tokens equal greedy_tokens and
its logits are within 1e-4 of greedy_logits, in eager calls and in replays of a captured graph, at
self-KV buckets 64 and 128; mask layouts the step cannot express raise."""
import json
import os

import numpy as np
import pytest
import torch

from speech_serving import native
from speech_serving.models import WhisperClassSpeechEncoderDecoderModel

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "whisper_tiny_golden.npz")
SLOTS, SLOT, T_MAX = 3, 1, 32


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN, allow_pickle=False)
    cfg = json.loads(bytes(z["config_json"]).decode())
    state = {k[len("param."):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param.")}
    return z, cfg, state


class Buffers:
    """The static buffers GraphDecodeBuffers hands to decode_step_graph_fixed, for one bucket."""

    def __init__(self, z, cfg, cuda, bucket):
        L, H = cfg["num_decoder_layers"], cfg["num_heads"]
        D = cfg["hidden_dim"] // H
        g = torch.Generator().manual_seed(5)
        self.bucket = bucket
        self.self_kv = torch.zeros(SLOTS, L, 2, H, bucket, D, device=cuda)
        # idle slots hold unrelated data: none of it may reach the active slot
        self.cross_kv = torch.randn(SLOTS, L, 2, H, T_MAX, D, generator=g).to(cuda)
        self.t_enc = z["enc_k0"].shape[2]
        for l in range(L):
            self.cross_kv[SLOT, l, 0, :, :self.t_enc] = torch.from_numpy(z[f"enc_k{l}"][0]).to(cuda)
            self.cross_kv[SLOT, l, 1, :, :self.t_enc] = torch.from_numpy(z[f"enc_v{l}"][0]).to(cuda)
        self.token_ids = torch.ones(SLOTS, 1, dtype=torch.long, device=cuda)
        self.positions = torch.zeros(SLOTS, 1, dtype=torch.long, device=cuda)
        self.out = torch.zeros(SLOTS, dtype=torch.long, device=cuda)
        self.attn_mask = torch.full((SLOTS, 1, 1, bucket), -10000.0, device=cuda)
        self.cross_mask = torch.full((SLOTS, 1, 1, T_MAX), -10000.0, device=cuda)
        self.cross_mask[SLOT, 0, 0, :self.t_enc] = 0.0

    def set_step(self, token, pos):
        """prepare_replay for the active slot: its token, its position, keys 0..pos kept."""
        self.token_ids[SLOT, 0] = token
        self.positions[SLOT, 0] = pos
        self.attn_mask[SLOT].fill_(-10000.0)
        self.attn_mask[SLOT, 0, 0, :pos + 1] = 0.0

    def call(self, m):
        m.decode_step_graph_fixed(self.token_ids, self.positions, self.self_kv, self.cross_kv, self.out,
                                  self.bucket, SLOTS, g_attn_mask=self.attn_mask, g_cross_mask=self.cross_mask)


def golden_model(golden, cuda):
    z, cfg, state = golden
    m = WhisperClassSpeechEncoderDecoderModel(cfg["num_encoder_layers"], cfg["num_decoder_layers"], cfg["num_heads"],
                                              cfg["hidden_dim"], cfg["mel_dim"], cfg["vocab_size"])
    m.load_state_dict(state)
    return m.to(cuda).eval()


def inputs(z, cfg):
    """The tokens fed step by step (prompt, then the golden greedy tokens) and the steps whose
    outputs are the golden greedy steps."""
    seq = list(cfg["prompt"]) + z["greedy_tokens"].tolist()[:-1]
    return seq, len(cfg["prompt"]) - 1


@pytest.mark.parametrize("bucket", [64, 128])
def test_graph_fixed_step_matches_reference_golden(golden, cuda, bucket):
    z, cfg, _ = golden
    m = golden_model(golden, cuda)
    buf = Buffers(z, cfg, cuda, bucket)
    logits = []
    hook = m.lm_head.register_forward_hook(lambda mod, inp, out: logits.append(out[SLOT].detach().float().cpu()))
    seq, first = inputs(z, cfg)
    toks = []
    with torch.no_grad():
        for pos, tok in enumerate(seq):
            buf.set_step(tok, pos)
            buf.call(m)
            toks.append(int(buf.out[SLOT]))
    hook.remove()
    assert toks[first:] == z["greedy_tokens"].tolist()
    np.testing.assert_allclose(torch.stack(logits[first:]).numpy(), z["greedy_logits"], rtol=1e-4, atol=1e-4)
    # the slot's self-KV bucket holds the prompt K/V the reference's prefill produces
    for l in range(cfg["num_decoder_layers"]):
        got = buf.self_kv[SLOT, l, 0, :, :len(cfg["prompt"])].cpu().numpy()
        np.testing.assert_allclose(got, z[f"prefill_k{l}"][0], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("bucket", [64, 128])
def test_graph_fixed_step_in_a_captured_graph(golden, cuda, bucket):
    """Captured once, replayed once per step with the inputs rewritten in place (graph_decode_buffers.py
    :389-463): the slot's tokens equal the golden greedy tokens on every replay, with eager work and
    synchronisations between the replays."""
    z, cfg, _ = golden
    m = golden_model(golden, cuda)
    buf = Buffers(z, cfg, cuda, bucket)
    seq, first = inputs(z, cfg)
    native.reserve_attention(SLOTS, cfg["num_heads"], cfg["hidden_dim"] // cfg["num_heads"], max(bucket, T_MAX),
                             torch.float32, cuda)
    with torch.no_grad():
        buf.set_step(seq[0], 0)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            buf.call(m)  # warm-up outside the capture (allocations, workspace)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        buf.self_kv.zero_()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            buf.call(m)
        toks = []
        for pos, tok in enumerate(seq):
            buf.set_step(tok, pos)
            g.replay()
            torch.cuda.synchronize()
            toks.append(int(buf.out[SLOT]))
    assert toks[first:] == z["greedy_tokens"].tolist()


def test_graph_fixed_rejects_masks_it_cannot_express(golden, cuda):
    z, cfg, _ = golden
    m = golden_model(golden, cuda)
    buf = Buffers(z, cfg, cuda, 64)
    buf.set_step(cfg["prompt"][0], 3)
    buf.attn_mask[SLOT, 0, 0, 1] = -10000.0  # a hole inside the kept prefix
    with torch.no_grad(), pytest.raises(ValueError, match="prefix"):
        buf.call(m)
    buf.set_step(cfg["prompt"][0], 3)
    buf.cross_mask[SLOT, 0, 0, 2] = -0.5  # a bias, not a mask
    with torch.no_grad(), pytest.raises(NotImplementedError):
        buf.call(m)
