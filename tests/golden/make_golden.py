"""Write golden vectors of the reference's synthetic Whisper-class model.

Run in the development container, where the reference repository is mounted:
    python tests/golden/make_golden.py [/path/to/reference]          # float32 vectors
    python tests/golden/make_golden.py [/path/to/reference] --lowp   # fp16 / bf16 greedy decodes

--lowp writes tests/golden/whisper_lowp_golden.npz: the reference's own reduced-precision greedy
decode (its model in float16 and in bfloat16 on the CPU, decode_step with a DynamicCache, torch.argmax
per step) for four shapes, the golden tiny shape, a Whisper-tiny-like decoder (4 layers, d_model 384,
4 heads x 64), a base-shaped (6 layers, 512, 8 x 64) and a small-shaped one (12 layers, 768, 12 x 64), the
last three with vocab 51865, 1500 encoder positions and the Whisper prompt, two requests each: per step the
token and the top-16 logits (index, value); for the tiny shape every logit. Weights and encoder K/V are
regenerated from seeds by name (oracle/rounding.seeded_state / seeded_cross_kv); the file records their
checksums so a run that regenerates them can check it has the same inputs.

The float32 mode:
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


LOWP_OUT = os.path.join(HERE, "whisper_lowp_golden.npz")
LOWP_SHAPES = {
    # layers, heads, hidden, head_dim, vocab, encoder positions, prompt, steps, weight std, K/V std, seeds
    "tiny": dict(layers=2, heads=2, hidden=32, head_dim=16, vocab=100, t_enc=20, prompt=[1, 2, 3], steps=24,
                 std=0.1, kv_std=1.0, seed=2101, kv_seeds=[2102, 2103]),
    "c1": dict(layers=4, heads=4, hidden=384, head_dim=64, vocab=51865, t_enc=1500,
               prompt=[50258, 50259, 50359, 50363], steps=32, std=0.02, kv_std=0.4, seed=2201,
               kv_seeds=[2202, 2203]),
    # the base-shaped (6 layers, 512, 8 x 64) and small-shaped (12 layers, 768, 12 x 64) decoders of the
    # serving scenarios
    "c3": dict(layers=6, heads=8, hidden=512, head_dim=64, vocab=51865, t_enc=1500,
               prompt=[50258, 50259, 50359, 50363], steps=24, std=0.02, kv_std=0.4, seed=2301,
               kv_seeds=[2302, 2303]),
    "c4": dict(layers=12, heads=12, hidden=768, head_dim=64, vocab=51865, t_enc=1500,
               prompt=[50258, 50259, 50359, 50363], steps=24, std=0.03, kv_std=0.4, seed=2401,
               kv_seeds=[2402, 2403]),
}
LOWP_DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}
TOPK = 16


def lowp_model(ref_models, cfg, dtype):
    """The reference model of a LOWP_SHAPES entry with its seeded weights, cast to dtype; (model, state)."""
    sys_layer = ref_models.DecoderLayer
    model = ref_models.WhisperClassSpeechEncoderDecoderModel(
        num_encoder_layers=0, num_decoder_layers=cfg["layers"], num_heads=cfg["heads"],
        hidden_dim=cfg["hidden"], mel_dim=80, vocab_size=cfg["vocab"])
    if cfg["hidden"] // cfg["heads"] != cfg["head_dim"]:  # layers built with an explicit head_dim
        model.decoder_layers = torch.nn.ModuleList(
            [sys_layer(cfg["hidden"], cfg["heads"], cfg["head_dim"], is_decoder=True) for _ in range(cfg["layers"])])
        model.head_dim = cfg["head_dim"]
    from oracle.rounding import seeded_state  # noqa: E402

    state = seeded_state({k: tuple(v.shape) for k, v in model.state_dict().items()}, cfg["seed"], cfg["std"])
    model.load_state_dict(state)
    return model.to(dtype).eval(), state


def write_lowp(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # the repository root, for oracle/
    import speech_serving.models as ref_models  # noqa: E402  (reference)

    from oracle.rounding import checksums, seeded_cross_kv  # noqa: E402

    out = {}
    summary = []
    for shape, cfg in LOWP_SHAPES.items():
        for dname, dtype in LOWP_DTYPES.items():
            model, state = lowp_model(ref_models, cfg, dtype)
            out[f"{shape}.{dname}.param_checksums"] = checksums({k: v.to(dtype) for k, v in state.items()}).numpy()
            for r, kv_seed in enumerate(cfg["kv_seeds"]):
                cross = [(k.to(dtype), v.to(dtype)) for k, v in
                         seeded_cross_kv(cfg["layers"], cfg["heads"], cfg["t_enc"], cfg["head_dim"], kv_seed,
                                         cfg["kv_std"])]
                key = f"{shape}.{dname}.r{r}"
                out[f"{key}.kv_checksums"] = checksums({f"{l}.{j}": t for l, kv in enumerate(cross)
                                                        for j, t in enumerate(kv)}).numpy()
                toks, tk_i, tk_v, full = [], [], [], []
                with torch.no_grad():
                    cur = model.decode_step(torch.tensor([cfg["prompt"]]), None, cross, use_cache=True)
                    for _ in range(cfg["steps"]):
                        last = cur.logits[:, -1, :]
                        vals, idx = torch.topk(last[0].float(), TOPK)
                        tk_i.append(idx.numpy())
                        tk_v.append(vals.numpy())
                        if shape == "tiny":
                            full.append(last[0].float().numpy())
                        t = int(torch.argmax(last, dim=-1).item())
                        toks.append(t)
                        cur = model.decode_step(torch.tensor([[t]]), cur.past_key_values, cross, use_cache=True)
                out[f"{key}.tokens"] = np.array(toks, dtype=np.int64)
                out[f"{key}.topk_idx"] = np.stack(tk_i).astype(np.int64)
                out[f"{key}.topk_val"] = np.stack(tk_v).astype(np.float32)
                if full:
                    out[f"{key}.logits"] = np.stack(full).astype(np.float32)
                summary.append((key, toks[:8]))
    out["config_json"] = np.frombuffer(json.dumps(dict(shapes=LOWP_SHAPES, dtypes=list(LOWP_DTYPES),
                                                       topk=TOPK)).encode(), dtype=np.uint8)
    np.savez_compressed(LOWP_OUT, **out)
    print(f"wrote {LOWP_OUT} ({os.path.getsize(LOWP_OUT)} bytes, {len(out)} arrays)")
    for key, toks in summary:
        print(f"  {key}: first tokens {toks}")


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    root = args[0] if args else "/root/reference"
    if "--lowp" in sys.argv[1:]:
        write_lowp(root)
    else:
        main(root)
