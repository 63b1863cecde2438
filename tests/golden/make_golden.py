"""Write golden vectors of the reference's synthetic Whisper-class model.

Run in the development container, where the reference repository is mounted:
    python tests/golden/make_golden.py [/path/to/reference]
It imports speech_serving.models from the reference (CPU, float32), builds a
tiny seeded model, and saves weights, inputs and outputs to
tests/golden/whisper_tiny_golden.npz (numpy arrays only, no pickles):
    encode(mel)                          -> enc_hidden, enc_k{l}, enc_v{l}
    decode_step(prompt, enc KV)          -> prefill_logits (+ self K/V per layer)
    greedy loop with the contiguous past  -> greedy_tokens, greedy_logits
    decode_step(prompt, encoder_hidden_states=...) -> proj_logits
The oracle (oracle/decoder.py) is checked against this file by
tests/test_decoder_oracle.py. No test, benchmark or library code reads the reference;
the tests read only this file.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "whisper_tiny_golden.npz")

CONFIG = dict(num_encoder_layers=2, num_decoder_layers=2, num_heads=2, hidden_dim=32, mel_dim=80, vocab_size=100)
SEED = 1234
MEL_LEN = 40
PROMPT = [1, 2, 3]
NEW_TOKENS = 8


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from speech_serving.models import WhisperClassSpeechEncoderDecoderModel  # noqa: E402  (reference)

    torch.manual_seed(SEED)
    model = WhisperClassSpeechEncoderDecoderModel(**CONFIG).eval()
    g = torch.Generator().manual_seed(SEED + 1)
    # Distinct LayerNorm parameters so norm1 / norm2 / norm3 are distinguishable.
    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, torch.nn.LayerNorm):
                mod.weight.add_(0.2 * torch.randn(mod.weight.shape, generator=g))
                mod.bias.add_(0.2 * torch.randn(mod.bias.shape, generator=g))
    mel = torch.randn(1, CONFIG["mel_dim"], MEL_LEN, generator=g)
    out = {f"param.{k}": v.detach().numpy().copy() for k, v in model.state_dict().items()}
    out["mel"] = mel.numpy()
    with torch.no_grad():
        hidden, enc_kv = model.encode(mel)
        out["enc_hidden"] = hidden.numpy()
        for l, (k, v) in enumerate(enc_kv):
            out[f"enc_k{l}"] = k.numpy()
            out[f"enc_v{l}"] = v.numpy()
        prompt = torch.tensor([PROMPT])
        pre = model.decode_step(prompt, None, enc_kv, use_cache=True)
        out["prefill_logits"] = pre.logits.numpy()
        for l in range(CONFIG["num_decoder_layers"]):
            out[f"prefill_k{l}"] = pre.past_key_values.layers[l].keys.numpy()
            out[f"prefill_v{l}"] = pre.past_key_values.layers[l].values.numpy()
        # greedy loop exactly as test_speech_engine.py:264-280, but from the prompt
        toks, logits = [], []
        cur = pre
        for _ in range(NEW_TOKENS):
            last = cur.logits[:, -1, :]
            logits.append(last[0].numpy())
            t = int(torch.argmax(last, dim=-1).item())
            toks.append(t)
            cur = model.decode_step(torch.tensor([[t]]), cur.past_key_values, enc_kv, use_cache=True)
        out["greedy_tokens"] = np.array(toks, dtype=np.int64)
        out["greedy_logits"] = np.stack(logits)
        proj = model.decode_step(prompt, None, None, encoder_hidden_states=hidden, use_cache=True)
        out["proj_logits"] = proj.logits.numpy()
    out["config_json"] = np.frombuffer(json.dumps(dict(CONFIG, seed=SEED, prompt=PROMPT,
                                                       new_tokens=NEW_TOKENS)).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays), greedy tokens {toks}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
